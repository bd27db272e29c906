#!/usr/bin/env python3
"""Render benchmark of the MI355X NeRF backend.

Workload (one step = one full inference render, inputs resident in HBM):
  analytic scene of 32 isotropic Gaussians (centres U[0.2,0.8]^3, sigma
  U(0.02,0.1), amplitude U(5,50), seed 0) -> 128^3 occupancy bitfield at
  density > 0.01; hash grid 16 levels x 2 fp16 features, T = 2^19, N_min 16,
  b 1.3819; density MLP 32->64->16 (exp), colour MLP SH4+geo -> 64 -> 64 -> 3
  (sigmoid), weights random-init (no checkpoint available offline); one
  800x800 view, pinhole f = 1111 px, pose on the radius-1.32 orbit around
  (0.5,0.5,0.5) (radius 4 in the Blender frame scaled by 0.33), <= 1024
  march steps per ray, early stop at transmittance < 1e-4.

Metric: Mrays/s = 640,000 rays / render time (whole pipeline: march count,
scan, march samples, fused field, composite; the one host sync for the sample
total is inside the timed region).  Alongside: the roofline of the dominant
kernel (the fused field kernel, HBM-bound by its algorithmic bytes) timed with
HIP events on the render stream, and the scalar CPU oracle timed on a bounded
ray subset of the same view on the host cores.

Training (reported in the same line as "train"): 100 800x800 target views of
the same scene rendered on the GPU from seeded poses on the same orbit; each
step marches a batch whose ray count adapts to 2^18 samples (hard cap 2^18),
Huber loss, full backward through composite, MLPs and hash grid, Adam (lr
1e-2, betas 0.9/0.99, eps 1e-15, loss scale 128), occupancy refresh every 16
steps with decay 0.95.  Train samples/s = samples trained on in the timed
steps / wall time of those steps.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--train-steps K2]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, GB/s
MFMA_FP16_PEAK_TFS = 2500.0  # MI355X dense fp16 MFMA, TFLOP/s
W = H = 800
FOCAL = 1111.0
MAX_STEPS = 1024
T_STOP = 1e-4
CENTRE = (0.5, 0.5, 0.5)
RADIUS = 1.32
TRAIN_W = TRAIN_H = 800
# Algorithmic bytes of the fused field kernel per sample: sample record
# (t_mid, dt, ray id) 12 B + 16 levels x 8 corners x 2 fp16 features 512 B +
# (sigma, r, g, b) fp32 16 B.
FIELD_BYTES_PER_SAMPLE = 12 + 16 * 8 * 2 * 2 + 16
# Algorithmic MLP flops per sample: density 32x64 + 64x16, colour 31x64 +
# 64x64 + 64x3, two flops per multiply-add.
FIELD_FLOPS_PER_SAMPLE = 2 * (32 * 64 + 64 * 16) + 2 * (31 * 64 + 64 * 64 + 64 * 3)
# Traffic beyond L2 of the field kernel per sample on this workload, from
# rocprofv3 FETCH_SIZE (x 2.0) + WRITE_SIZE (x 1.0) on one 800x800 render, the
# factors being what the same counters read on a plain conversion kernel of
# known size (profiles/field_forward_800x800_counters.md): 217.52 GB + 7.83 GB
# over 486,308,861 samples, summed over the render's dispatches.  The render
# rounds list samples in spatial order, so neighbouring lanes share the coarse
# levels' table lines and the traffic stays near the 540 algorithmic bytes
# (58 % L2 hit).
FIELD_TRAFFIC_BYTES_PER_SAMPLE = 463
# Reference-model network per sample, on the reference's own padded shapes
# (backend-cuda.cu:23-54): density 64x128 + 4 x 128x128 + 128x16, colour
# 48x128 + 2 x 128x128 + 128x16, two flops per multiply-add.
REF_FLOPS_PER_SAMPLE = 2 * (64 * 128 + 4 * 128 * 128 + 128 * 16) + 2 * (48 * 128 + 2 * 128 * 128 + 128 * 16)
# Its MLP backward per sample: the forward recomputed (233,472), input
# gradients of every layer but the density input (density 2 x (16x128 +
# 4 x 128x128), colour 2 x (16x128 + 2 x 128x128), the colour input's 15
# geometry columns 2 x 15x128: 208,640) and the weight gradients (233,472).
REF_BACKWARD_FLOPS_PER_SAMPLE = REF_FLOPS_PER_SAMPLE + 2 * (16 * 128 + 4 * 128 * 128) + 2 * (16 * 128 + 2 * 128 * 128) + 2 * 15 * 128 + REF_FLOPS_PER_SAMPLE


def build_workload():
    from nerf_amd import _lib as L, ext

    scene = ext.scene_gaussians(32, seed=0)
    bits = ext.occupancy_from_scene(scene, 128, threshold=0.01)
    desc = ext.grid_desc(19, L.NERF_EXT_F16)
    model = ext.Model.create(desc, seed=0)
    cam = ext.camera_orbit(0, 0, RADIUS, CENTRE, W, H, FOCAL * W / 800.0)  # field of view of the 800-px view
    occ = ext.occupancy_struct(bits, 128)
    return scene, bits, desc, model, cam, occ


# Hash-encode forward, 16 levels x 2 fp32 features, T = 2^16: position 12 B
# + 16 levels x 8 corners x 2 features x 4 B + 32 fp32 outputs = 1,164 B/point.
ENCODE_BYTES_PER_POINT = 12 + 16 * 8 * 2 * 4 + 32 * 4


def unit_points(n: int, seed: int) -> np.ndarray:
    """n points in [0,1)^3: draws 0..3n-1 of the library's splitmix64 stream
    keyed (0x9017, seed), 24-bit uniforms (the points of the parity tests)."""
    m = np.uint64(0xFFFFFFFFFFFFFFFF)
    golden, mix1, mix2 = np.uint64(0x9E3779B97F4A7C15), np.uint64(0xBF58476D1CE4E5B9), np.uint64(0x94D049BB133111EB)
    with np.errstate(over="ignore"):
        state0 = (np.uint64(0x9017) + golden) ^ (np.uint64(seed) * mix1)
        z = state0 + (np.arange(3 * n, dtype=np.uint64) + np.uint64(1)) * golden
        z = (z ^ (z >> np.uint64(30))) * mix1
        z = (z ^ (z >> np.uint64(27))) * mix2
        z = (z ^ (z >> np.uint64(31))) & m
    u = ((z >> np.uint64(40)).astype(np.float32)) * np.float32(1.0 / 16777216.0)
    return u.reshape(n, 3)


def kernel_rooflines(reps_small: int = 200):
    """Stage rooflines of the hash encode (HBM) and the fused MLP (MFMA)."""
    from nerf_amd import _lib as L, ext
    from nerf_amd.device import DeviceArray, Event, Stream
    out = {}
    st = Stream()

    def timed(fn, reps):
        fn()
        st.synchronize()
        e0, e1 = Event(), Event()
        e0.record(st)
        for _ in range(reps):
            fn()
        e1.record(st)
        st.synchronize()
        return e0.elapsed_ms(e1) / reps

    desc = ext.grid_desc(16, L.NERF_EXT_F32)
    table = ext.init_table(desc, 0, 1e-4)
    for n, reps, label in ((1 << 16, reps_small, "encode_forward_2p16"), (1 << 24, 20, "encode_forward_2p24")):
        pos = DeviceArray.from_numpy(unit_points(n, seed=0))
        feats = DeviceArray((n, 32), np.float32)
        ms = timed(lambda: L.call("nerf_ext_encode_forward", C.byref(desc), table.ptr, pos.ptr, n, feats.ptr, L.NERF_EXT_F32, st.handle), reps)
        gbs = n * ENCODE_BYTES_PER_POINT / (ms / 1e3) / 1e9
        out[label] = {"kernel": "k_encode_split (nerf_ext_encode_forward, four levels per XCD, one point per thread)", "points": n, "table": "16 x 2^16 x 2 fp32", "ms": round(ms, 5), "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_point": ENCODE_BYTES_PER_POINT, "reps": reps}
    rng = np.random.default_rng(0)
    dp = DeviceArray.from_numpy(ext.mlp_init(0).astype(np.float16))
    cp = DeviceArray.from_numpy(ext.mlp_init(1).astype(np.float16))
    for n, label in ((1 << 22, "field_mlp"), (1 << 24, "field_mlp_2p24")):
        feats = DeviceArray.from_numpy(rng.uniform(-1.0, 1.0, size=(n, 32)).astype(np.float16))
        d = rng.normal(size=(n, 3)).astype(np.float32)
        dirs = DeviceArray.from_numpy(d / np.linalg.norm(d, axis=1, keepdims=True))
        res = DeviceArray((n, 4), np.float32)
        ms = timed(lambda: L.call("nerf_ext_field_mlp", dp.ptr, cp.ptr, feats.ptr, dirs.ptr, n, res.ptr, st.handle), 20)
        tfs = n * FIELD_FLOPS_PER_SAMPLE / (ms / 1e3) / 1e12
        io_gbs = n * (64 + 12 + 16) / (ms / 1e3) / 1e9
        out[label] = {"kernel": "k_field_mlp (density 32-64-16 + colour 32-64-64-16, fp16 MFMA)", "samples": n, "ms": round(ms, 4), "bound": "mfma", "achieved": round(tfs, 1), "peak": MFMA_FP16_PEAK_TFS, "unit": "TFLOP/s",
                      "frac": round(tfs / MFMA_FP16_PEAK_TFS, 4), "flops_per_sample": FIELD_FLOPS_PER_SAMPLE, "io_GBps": round(io_gbs, 1)}
        del feats, dirs, res
    # Reference-model field (frequency encoding + the reference's 128-wide
    # MLPs, fused), 2^22 world points in [-1.5, 1.5]^3.
    rm = ext.RefModel.create()
    n = 1 << 22
    p = rng.uniform(-1.5, 1.5, size=(n, 3)).astype(np.float32)
    d = rng.normal(size=(n, 3)).astype(np.float32)
    pos, dirs = DeviceArray.from_numpy(p), DeviceArray.from_numpy(d / np.linalg.norm(d, axis=1, keepdims=True))
    res = DeviceArray((n, 4), np.float32)
    ms = timed(lambda: L.call("nerf_ext_ref_field_forward", rm.density.ptr, rm.color.ptr, pos.ptr, dirs.ptr, n, res.ptr, None, st.handle), 20)
    tfs = n * REF_FLOPS_PER_SAMPLE / (ms / 1e3) / 1e12
    nb = 1 << 18
    draw = DeviceArray.from_numpy(rng.normal(0, 1e-2, size=(nb, 4)).astype(np.float32))
    gD, gC = DeviceArray((L.NERF_EXT_REF_DENSITY_PARAMS,), np.float32), DeviceArray((L.NERF_EXT_REF_COLOR_PARAMS,), np.float32)
    ms_b = timed(lambda: L.call("nerf_ext_ref_backward", rm.density.ptr, rm.color.ptr, pos.ptr, dirs.ptr, draw.ptr, nb, 128.0, gD.ptr, gC.ptr, st.handle), 20)
    tfs_b = nb * REF_BACKWARD_FLOPS_PER_SAMPLE / (ms_b / 1e3) / 1e12
    out["ref_backward_2p18"] = {"kernel": "k_ref_backward + k_ref_dw + k_ref_dw_reduce (reference-model MLP backward: recompute, deltas, weight gradients)", "samples": nb, "ms": round(ms_b, 4), "bound": "mfma",
                                "achieved": round(tfs_b, 1), "peak": MFMA_FP16_PEAK_TFS, "unit": "TFLOP/s", "frac": round(tfs_b / MFMA_FP16_PEAK_TFS, 4), "flops_per_sample": REF_BACKWARD_FLOPS_PER_SAMPLE}
    out["ref_field_2p22"] = {"kernel": "k_ref_field (reference-model mode: frequency encoding, density 64-128x5-16, colour 48-128x3-16, fp16 MFMA)", "samples": n, "ms": round(ms, 4), "bound": "mfma", "achieved": round(tfs, 1),
                             "peak": MFMA_FP16_PEAK_TFS, "unit": "TFLOP/s", "frac": round(tfs / MFMA_FP16_PEAK_TFS, 4), "flops_per_sample": REF_FLOPS_PER_SAMPLE}
    return out


def ref_model_render(reps: int = 3):
    """The headline 800x800 render with the reference's own network in place
    of the hash-grid model (reference-model mode, the reference's init)."""
    from nerf_amd import ext
    from nerf_amd.device import synchronize
    scene, bits, desc, model, cam, occ = build_workload()
    rm = ext.RefModel.create()
    r = ext.Renderer()
    r.render(rm, occ, [cam], MAX_STEPS, T_STOP)
    synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        _, st = r.render(rm, occ, [cam], MAX_STEPS, T_STOP, timed=True)
    wall = (time.perf_counter() - t0) / reps
    tfs = st.samples_shaded * REF_FLOPS_PER_SAMPLE / (st.ms_field / 1e3) / 1e12
    return {"value": round(W * H / wall / 1e6, 3), "unit": "Mrays/s", "ms_per_render": round(wall * 1e3, 2), "field_ms": round(st.ms_field, 2), "samples_shaded": int(st.samples_shaded),
            "field_tflops": round(tfs, 1), "field_mfma_frac": round(tfs / MFMA_FP16_PEAK_TFS, 4), "reps": reps,
            "workload": "800x800, 32-Gaussian scene, 128^3 occupancy, <=1024 steps/ray, reference-model network (frequency encoding, 128-wide MLPs, softplus)"}


def train_bench(steps: int, warmup: int, views: int = 100):
    """Training throughput on the analytic scene (2^18-sample batches)."""
    from nerf_amd import _lib as L, ext
    from nerf_amd.device import Event

    scene = ext.scene_gaussians(32, seed=0)
    cams = [ext.camera_orbit(1, i, RADIUS, CENTRE, TRAIN_W, TRAIN_H, FOCAL) for i in range(views)]
    images = ext.scene_render(scene, cams, 512).numpy()
    desc = ext.grid_desc(19, L.NERF_EXT_F16)
    hyper = ext.hyper_params(lr=1e-2, beta1=0.9, beta2=0.99, eps=1e-15, loss_scale=128.0)
    occ = ext.occupancy_params(decay=0.95, threshold=0.01, cells_per_update=128 ** 3, update_interval=16, warmup_steps=16)
    batch = 1 << 18
    tr = ext.Trainer(desc, images.view(np.uint8), cams, occupancy_res=128, hyper=hyper, occupancy=occ, initial_rays=4096, max_rays=batch, target_samples=batch, sample_capacity=batch,
                     max_steps_per_ray=MAX_STEPS, seed=0)
    del images

    class _On:
        handle = tr.stream()

    tr.step(warmup)
    s0 = tr.stats()
    ev0, ev1 = Event(), Event()
    t0 = time.perf_counter()
    ev0.record(_On)
    tr.step(steps)
    ev1.record(_On)
    s1 = tr.stats()  # synchronises the trainer's stream
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_ms(ev1)
    samples = s1.samples_total - s0.samples_total
    out = {"samples_per_s": round(samples / wall, 1), "unit": "train samples/s", "steps": steps, "warmup": warmup, "ms_per_step": round(wall * 1e3 / steps, 4),
           "gpu_ms_per_step": round(gpu_ms / steps, 4), "mean_samples_per_step": round(samples / steps, 1), "rays_last_step": s1.rays, "loss_first_timed": None,
           "loss_last": round(float(s1.last.loss), 6), "nonfinite": int(s1.last.has_nonfinite), "batch_target": batch, "views": views,
           "workload": f"{views} 800x800 views, 32-Gaussian scene, hash grid T=2^19 fp16, 128^3 occupancy, 2^18-sample batches, <=1024 steps/ray"}
    out["loss_first_timed"] = round(float(s0.last.loss), 6)
    out["stages"] = train_stages(tr, _On, reps=20)
    out["render_trained"] = render_trained(tr)
    snap = train_snapshot(tr, cams, scene)
    tr.close()
    return out, snap


def train_snapshot(tr, cams, scene):
    """The inputs of the trainer's next step, for the CPU oracle's timing of
    the same step: step index, ray count, picked camera and its image, the
    occupancy and the model."""
    from nerf_amd import _lib as L, ext
    from oracle import oracle as orc
    st = tr.stats()
    frame = st.last.completed_steps
    view = orc.train_camera(frame, len(cams))
    image = ext.scene_render(scene, [cams[view]], 512).numpy()[0].view(np.uint8)
    m, _ = tr.model()
    B = tr.buffers()
    E = int(B.table_elems)
    return {"frame": frame, "rays": int(st.rays), "cam": cams[view], "ocam": orc.camera_from_bytes(bytes(cams[view])), "image": np.ascontiguousarray(image),
            "bits": ext.read_device(B.bitfield, (128 ** 3 // 32,), np.uint32), "grid": orc.make_grid(16, 19, 1), "table": ext.read_device(m.table, (E,), np.uint16),
            "table32": ext.read_device(B.table_f32, (E,), np.float32), "dp": ext.read_device(m.density_params, (L.NERF_EXT_DENSITY_PARAMS,), np.uint16),
            "cp": ext.read_device(m.color_params, (L.NERF_EXT_COLOR_PARAMS,), np.uint16)}


def ref_train_bench(steps: int, warmup: int, views: int = 100):
    """Training the reference's own network (frequency encoding, 128-wide
    MLPs, softplus, its alpha-weighted loss) in the trainer on the training
    leg's data and batch (2^18 samples, <=1024 steps/ray)."""
    from nerf_amd import _lib as L, ext
    from nerf_amd.device import Event

    scene = ext.scene_gaussians(32, seed=0)
    cams = [ext.camera_orbit(1, i, RADIUS, CENTRE, TRAIN_W, TRAIN_H, FOCAL) for i in range(views)]
    images = ext.scene_render(scene, cams, 512).numpy()
    hyper = ext.hyper_params(lr=5e-4, beta1=0.9, beta2=0.99, eps=1e-15, loss_scale=128.0)
    occ = ext.occupancy_params(decay=0.95, threshold=0.01, cells_per_update=128 ** 3, update_interval=16, warmup_steps=16)
    batch = 1 << 18
    tr = ext.Trainer(ext.grid_desc(19, L.NERF_EXT_F16), images.view(np.uint8), cams, occupancy_res=128, hyper=hyper, occupancy=occ, initial_rays=4096, max_rays=batch, target_samples=batch,
                     sample_capacity=batch, max_steps_per_ray=MAX_STEPS, seed=0, model_kind=L.NERF_EXT_MODEL_REFERENCE)
    del images

    class _On:
        handle = tr.stream()

    tr.step(warmup)
    s0 = tr.stats()
    t0 = time.perf_counter()
    tr.step(steps)
    s1 = tr.stats()
    wall = time.perf_counter() - t0
    n = (s1.samples_total - s0.samples_total) / steps
    groups = [("sample", L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_SAMPLE), ("forward", L.NERF_EXT_STAGE_FORWARD, L.NERF_EXT_STAGE_FORWARD), ("composite", L.NERF_EXT_STAGE_COMPOSITE, L.NERF_EXT_STAGE_COMPOSITE),
              ("backward", L.NERF_EXT_STAGE_BACKWARD, L.NERF_EXT_STAGE_BACKWARD), ("adam", L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)]
    reps = 10
    evs = [[Event() for _ in range(len(groups) + 1)] for _ in range(reps)]
    for r in range(reps):
        evs[r][0].record(_On)
        for k, (_, a, b) in enumerate(groups):
            tr.run_stages(a, b)
            evs[r][k + 1].record(_On)
    tr.stats()
    ms = {name: sum(evs[r][k].elapsed_ms(evs[r][k + 1]) for r in range(reps)) / reps for k, (name, _, _) in enumerate(groups)}
    params = L.NERF_EXT_REF_DENSITY_PARAMS + L.NERF_EXT_REF_COLOR_PARAMS

    def mfma(f, t):
        return {"achieved": round(f / (t / 1e3) / 1e12, 1), "unit": "TFLOP/s", "frac": round(f / (t / 1e3) / 1e12 / MFMA_FP16_PEAK_TFS, 4), "bound": "mfma"}

    out = {"samples_per_s": round(n * steps / wall, 1), "unit": "train samples/s", "steps": steps, "warmup": warmup, "ms_per_step": round(wall * 1e3 / steps, 4), "mean_samples_per_step": round(n, 1),
           "loss_last": round(float(s1.last.loss), 6), "nonfinite": int(s1.last.has_nonfinite),
           "stages": {"sample_ms": round(ms["sample"], 4), "forward": {"ms": round(ms["forward"], 4), **mfma(n * REF_FLOPS_PER_SAMPLE, ms["forward"])}, "composite_ms": round(ms["composite"], 4),
                      "backward": {"ms": round(ms["backward"], 4), **mfma(n * REF_BACKWARD_FLOPS_PER_SAMPLE, ms["backward"])}, "adam_ms": round(ms["adam"], 4), "parameters": params},
           "workload": f"{views} 800x800 views, 32-Gaussian scene, the reference's network (frequency encoding, density 64-128x5-16, colour 48-128x3-16), 2^18-sample batches, <=1024 steps/ray"}
    tr.close()
    return out


def leg_in_child(leg: str, extra: list) -> dict:
    """One leg run by `bench.py --only LEG` in a child process of its own (a
    fresh HIP context), as the reference's benchmark program runs on its own;
    its JSON result, with the process noted."""
    import subprocess
    proc = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", leg, *extra], capture_output=True, text=True, timeout=900)
    lines = [x for x in proc.stdout.splitlines() if x.startswith('{"leg"')]
    if proc.returncode != 0 or not lines:
        raise RuntimeError(f"bench.py --only {leg} failed ({proc.returncode}): {proc.stderr[-2000:]}")
    result = json.loads(lines[-1])["result"]
    result["process"] = "a child process of its own (bench.py --only " + " ".join([leg, *extra]) + "), as benchmark.cpp runs"
    return result


def reference_host_bench(steps: int = 200, views: int = 100):
    """The reference host program's workload (benchmark.cpp:305-546) through
    nerf.h with the reference's own network: 4,096 rays per step, <= 64
    steps per ray, its hyper-parameters and occupancy schedule; the metric it
    prints, steps/s, and nerf_inference at its 64 samples per ray (the
    reference's uniform sampling)."""
    from nerf_amd import _lib as L, ext

    scene = ext.scene_gaussians(32, seed=0)
    cams = [ext.camera_orbit(1, i, RADIUS, CENTRE, TRAIN_W, TRAIN_H, FOCAL) for i in range(views)]
    images = np.ascontiguousarray(ext.scene_render(scene, cams, 512).numpy())
    mats = np.zeros((views, 4, 4), np.float32)
    for i, c in enumerate(cams):
        mats[i, :3, :] = np.array(c.c2w[:], np.float32).reshape(3, 4)
        mats[i, 3, 3] = 1.0
    d = L.NerfCreateDesc(128, 1 << 21, 1 << 16, 256, images.ctypes.data, images.nbytes, mats.ctypes.data, mats.nbytes, views, TRAIN_W, TRAIN_H, cams[0].fx, cams[0].fy, cams[0].cx, cams[0].cy)
    h = C.c_void_p()
    L.call("nerf_create_context", C.byref(d), C.byref(h))
    out = {}
    try:
        for name, kind in (("reference_model", L.NERF_EXT_MODEL_REFERENCE), ("hashgrid_model", L.NERF_EXT_MODEL_HASHGRID)):
            L.call("nerf_ext_context_configure", h, C.byref(L.NerfExtContextOptions(kind, L.NERF_EXT_SAMPLING_UNIFORM)))
            hp = L.NerfHyperParams(5e-4, 0.9, 0.999, 1e-8, 1.0, 100.0, 128.0, 250)
            occ = L.NerfOccupancyParams(0.98, 0.01, 65536, 1, 32)
            L.call("nerf_configure_training", h, C.byref(L.NerfTrainingConfig(0.0, 0.0, 0.0, 1.0, 1.0, 1.0, hp, occ, 4096, 64)))
            for _ in range(20):
                L.call("nerf_train_step", h)
            st = L.NerfTrainStats()
            L.call("nerf_read_train_stats", h, C.byref(st))
            t0 = time.perf_counter()
            for _ in range(steps):
                L.call("nerf_train_step", h)
            L.call("nerf_read_train_stats", h, C.byref(st))
            wall = time.perf_counter() - t0
            img = np.zeros((TRAIN_H, TRAIN_W), np.uint32)
            req = L.NerfInferenceRequest(0, 64, L.NERF_MEMORY_HOST, img.ctypes.data, img.nbytes)
            info = L.NerfInferenceInfo()
            L.call("nerf_inference", h, C.byref(req), C.byref(info))
            t1 = time.perf_counter()
            reps = 3
            for _ in range(reps):
                L.call("nerf_inference", h, C.byref(req), C.byref(info))
            iw = (time.perf_counter() - t1) / reps
            out[name] = {"sps": round(steps / wall, 2), "unit": "train steps/s", "rays_per_s": round(4096 * steps / wall, 1), "steps": steps, "loss_last": round(float(st.loss), 6),
                         "nonfinite": int(st.has_nonfinite), "inference_ms": round(iw * 1e3, 3), "inference_mrays_per_s": round(TRAIN_W * TRAIN_H / iw / 1e6, 3),
                         "inference": "nerf_inference, 64 uniform samples per ray over the box (the reference's sampling), RGBA8 to host"}
    finally:
        L.call("nerf_destroy_context", h)
    out["workload"] = f"benchmark.cpp defaults through nerf.h: {views} 800x800 views, 4096 rays/step, <=64 steps/ray, lr 5e-4, betas 0.9/0.999, eps 1e-8, clip 1, guard 100, loss scale 128, decay 250k; occupancy decay 0.98, 65536 cells/update every step after 32 warmup steps"
    return out


# Algorithmic work per training stage (per sample unless noted): the march
# writes a 16-byte sample and reads a 32-byte ray; the field forward gathers a
# 588-byte f16 encoding and runs 18,688 MLP flops; compositing reads and writes
# 44 bytes; the backward scatters the encoding gradient (2,124 bytes counting
# read-modify-write) and runs 37,376 MLP flops; Adam moves 30 bytes per
# parameter.
TRAIN_MARCH_B_SAMPLE, TRAIN_MARCH_B_RAY = 16, 32
TRAIN_ENCODE_B = 12 + 16 * 8 * 2 * 2 + 32 * 2
TRAIN_COMPOSITE_B = 44
TRAIN_ENC_BWD_B = 12 + 64 + 2 * (16 * 8 * 2 * 4)
TRAIN_BWD_FLOPS = 2 * FIELD_FLOPS_PER_SAMPLE
ADAM_B_PARAM = 30


def train_stages(tr, on, reps: int):
    """Per-stage times of `reps` further steps, each stage bracketed by HIP
    events on the trainer's stream, with each stage's roofline fraction."""
    from nerf_amd import _lib as L
    from nerf_amd.device import Event

    groups = [("sample", L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_SAMPLE), ("forward", L.NERF_EXT_STAGE_FORWARD, L.NERF_EXT_STAGE_FORWARD),
              ("composite", L.NERF_EXT_STAGE_COMPOSITE, L.NERF_EXT_STAGE_COMPOSITE), ("backward", L.NERF_EXT_STAGE_BACKWARD, L.NERF_EXT_STAGE_BACKWARD),
              ("adam", L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)]
    evs = [[Event() for _ in range(len(groups) + 1)] for _ in range(reps)]
    s0 = tr.stats()
    for r in range(reps):
        evs[r][0].record(on)
        for k, (_, a, b) in enumerate(groups):
            tr.run_stages(a, b)
            evs[r][k + 1].record(on)
    s1 = tr.stats()
    ms = {name: sum(evs[r][k].elapsed_ms(evs[r][k + 1]) for r in range(reps)) / reps for k, (name, _, _) in enumerate(groups)}
    n = (s1.samples_total - s0.samples_total) / reps
    rays = s1.rays
    params = 16 * (1 << 19) * 2 + 10240

    def hbm(b, t):
        return {"achieved": round(b / (t / 1e3) / 1e9, 1), "unit": "GB/s", "frac": round(b / (t / 1e3) / 1e9 / HBM_PEAK_GBS, 4), "bound": "hbm"}

    def mfma(f, t):
        return {"achieved": round(f / (t / 1e3) / 1e12, 1), "unit": "TFLOP/s", "frac": round(f / (t / 1e3) / 1e12 / MFMA_FP16_PEAK_TFS, 4), "bound": "mfma"}

    out = {"reps": reps, "samples_per_step": round(n, 1), "rays_last_step": rays,
           "sample": {"ms": round(ms["sample"], 4), **hbm(n * TRAIN_MARCH_B_SAMPLE + rays * TRAIN_MARCH_B_RAY, ms["sample"]), "work": "16 B/sample + 32 B/ray (march, scan, compaction; occupancy refresh every 16 steps)"},
           "forward": {"ms": round(ms["forward"], 4), **mfma(n * FIELD_FLOPS_PER_SAMPLE, ms["forward"]), "hbm": hbm(n * TRAIN_ENCODE_B, ms["forward"]), "work": "18,688 flop + 588 B/sample"},
           "composite": {"ms": round(ms["composite"], 4), **hbm(n * TRAIN_COMPOSITE_B, ms["composite"]), "work": "44 B/sample"},
           "backward": {"ms": round(ms["backward"], 4), **hbm(n * TRAIN_ENC_BWD_B, ms["backward"]), "mfma": mfma(n * TRAIN_BWD_FLOPS, ms["backward"]), "work": "2,124 B + 37,376 flop/sample"},
           "adam": {"ms": round(ms["adam"], 4), **hbm(params * ADAM_B_PARAM, ms["adam"]), "work": "30 B/parameter, 16.8 M parameters"}}
    return out


def abi_render(model_seed: int = 0, reps: int = 5):
    """The 800x800 render through the reference ABI's nerf_inference, timed by
    wall clock around the call (RGBA8 returned in host memory).  The context
    holds a random-init model and, before training is configured, no
    occupancy grid: every cell of the unit box counts as occupied, so this is
    a heavier workload than the headline render's 128^3 scene occupancy."""
    from nerf_amd import _lib as L, ext

    cam = ext.camera_orbit(0, 0, RADIUS, CENTRE, W, H, FOCAL)
    img = np.zeros((1, H, W), np.uint32)
    mat = np.zeros((1, 4, 4), np.float32)
    mat[0, :3, :] = np.array(cam.c2w[:], np.float32).reshape(3, 4)
    mat[0, 3, 3] = 1.0
    d = L.NerfCreateDesc(128, 1 << 20, 4096, 256, img.ctypes.data, img.nbytes, mat.ctypes.data, mat.nbytes, 1, W, H, cam.fx, cam.fy, cam.cx, cam.cy)
    h = C.c_void_p()
    L.call("nerf_create_context", C.byref(d), C.byref(h))
    try:
        out = np.zeros((H, W), np.uint32)
        req = L.NerfInferenceRequest(0, MAX_STEPS, L.NERF_MEMORY_HOST, out.ctypes.data, out.nbytes)
        info = L.NerfInferenceInfo()
        L.call("nerf_inference", h, C.byref(req), C.byref(info))
        t0 = time.perf_counter()
        for _ in range(reps):
            L.call("nerf_inference", h, C.byref(req), C.byref(info))
        wall = (time.perf_counter() - t0) / reps
    finally:
        L.call("nerf_destroy_context", h)
    return {"value": round(W * H / wall / 1e6, 3), "unit": "Mrays/s", "ms_per_render": round(wall * 1e3, 3), "reps": reps,
            "workload": f"{W}x{H} through nerf_inference (wall clock, RGBA8 to host): random-init model, every cell of the unit box occupied, <={MAX_STEPS} steps/ray"}


def render_trained(tr, reps: int = 5):
    """The 800x800 view rendered from the model the training leg produced
    (same scene, occupancy and camera as the headline render): rays retire
    once opaque, so only the samples in front of the first surface are
    shaded."""
    from nerf_amd import _lib as L, ext
    from nerf_amd.device import DeviceArray, Event, Stream, synchronize

    model, _ = tr.model()
    scene = ext.scene_gaussians(32, seed=0)
    bits = ext.occupancy_from_scene(scene, 128, threshold=0.01)
    occ = ext.occupancy_struct(bits, 128)
    cam = ext.camera_orbit(0, 0, RADIUS, CENTRE, TRAIN_W, TRAIN_H, FOCAL)
    rgba = DeviceArray((1, TRAIN_H, TRAIN_W), np.uint32)
    cams = (L.NerfExtCamera * 1)(cam)
    st = Stream()
    desc = L.NerfExtRenderDesc(C.pointer(model), C.pointer(occ), cams, 1, MAX_STEPS, T_STOP, (C.c_float * 3)(1.0, 1.0, 1.0), st.handle)
    r = ext.Renderer()
    L.call("nerf_ext_render", r._h, C.byref(desc), rgba.ptr, None, None, None)
    st.synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(reps):
        L.call("nerf_ext_render", r._h, C.byref(desc), rgba.ptr, None, None, None)
    e1.record(st)
    st.synchronize()
    wall = time.perf_counter() - t0
    stats = L.NerfExtRenderStats()
    L.call("nerf_ext_render", r._h, C.byref(desc), rgba.ptr, None, None, C.byref(stats))
    synchronize()
    return {"value": round(TRAIN_W * TRAIN_H / (wall / reps) / 1e6, 3), "unit": "Mrays/s", "ms_per_render": round(wall * 1e3 / reps, 3), "gpu_ms_per_render": round(e0.elapsed_ms(e1) / reps, 3),
            "samples_marched": int(stats.samples), "samples_shaded": int(stats.samples_shaded), "field_ms": round(stats.ms_field, 3), "reps": reps,
            "workload": "800x800 view of the trained model (analytic 128^3 occupancy, <=1024 steps/ray, early stop T<1e-4)"}


def config_renders(reps: int = 2):
    """The two large configurations as whole renders (one warm-up, then reps
    timed by wall clock around synchronised calls):
      C4: 1920x1080, hash grid T=2^22 fp16 with finest resolution 4096, 256
          Gaussians (as the headline scene), 256^3 occupancy, <=2048 steps/ray,
          focal 1111 * 1920 / 800 (the headline field of view);
      C5: 8 views of 1280x720 in one call (one compacted sample stream per
          chunk of rays), unbounded scene of 512 Gaussians over [-16, 16]^3
          (sigma U(0.3, 1.5), amplitude U(5, 50)) plus a uniform shell of radii
          12..15.5, 5 nested 128^3 cascades over [-1, 1]^3 .. [-16, 16]^3, hash
          grid T=2^21 fp16, <=4096 steps/ray, orbit radius 4, focal
          1111 * 1280 / 800.
    Random-init models, early stop at T < 1e-4."""
    from nerf_amd import _lib as L, ext
    from nerf_amd.device import synchronize

    def run(model, occ, cams, steps):
        r = ext.Renderer()
        r.render(model, occ, cams, steps, T_STOP)
        synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            _, st = r.render(model, occ, cams, steps, T_STOP, timed=True)
        wall = (time.perf_counter() - t0) / reps
        n = len(cams) * cams[0].width * cams[0].height
        return {"value": round(n / wall / 1e6, 3), "unit": "Mrays/s", "ms_per_render": round(wall * 1e3, 2), "field_ms": round(st.ms_field, 2), "samples_marched": int(st.samples),
                "samples_shaded": int(st.samples_shaded), "reps": reps}

    out = {}
    g = ext.scene_gaussians(256, seed=4)
    bits = ext.occupancy_from_scene(g, 256, 0.01)
    model = ext.Model.create(ext.grid_desc(22, L.NERF_EXT_F16, finest=4096), seed=0)
    cam = ext.camera_orbit(0, 0, RADIUS, CENTRE, 1920, 1080, FOCAL * 1920 / 800.0)
    out["C4"] = run(model, ext.occupancy_struct(bits, 256), [cam], 2048)
    out["C4"]["workload"] = "1920x1080, T=2^22 fp16 (finest 4096), 256 Gaussians, 256^3 occupancy, <=2048 steps/ray"
    del model, bits
    g = ext.scene_gaussians(512, seed=5, centre=(-16.0, 16.0), sigma=(0.3, 1.5), amplitude=(5.0, 50.0))
    bits = ext.occupancy_from_scene(g, 128, 0.01, (-1.0, -1.0, -1.0), (1.0, 1.0, 1.0), 5, shell=((0.0, 0.0, 0.0), 12.0, 15.5))
    model = ext.Model.create(ext.grid_desc(21, L.NERF_EXT_F16), seed=0)
    occ = ext.occupancy_struct(bits, 128, (-1.0, -1.0, -1.0), (1.0, 1.0, 1.0), 5)
    cams = [ext.camera_orbit(5, i, 4.0, (0.0, 0.0, 0.0), 1280, 720, FOCAL * 1280 / 800.0) for i in range(8)]
    out["C5"] = run(model, occ, cams, 4096)
    out["C5"]["workload"] = "8 x 1280x720 in one call, 5 x 128^3 cascades, 512 Gaussians over radius 16 + shell, T=2^21 fp16, <=4096 steps/ray"
    return out


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _split(n: int, parts: int):
    step = (n + parts - 1) // parts
    return [(b, min(n, b + step)) for b in range(0, n, step)]


def _threaded(fn, n: int, threads: int):
    """fn(begin, end) over `threads` slices of range(n) on Python threads (the
    oracle's ctypes calls release the GIL), results in slice order."""
    if threads <= 1:
        return [fn(0, n)]
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=threads) as ex:
        return list(ex.map(lambda be: fn(*be), _split(n, threads)))


def cpu_render_leg(model, cam, bits, threads: int, budget_s: float, gpu_image=None):
    """The scalar oracle's render (march + field + composite) on a
    deterministic ray subset of the headline view, sized to about budget_s.
    gpu_image = (rgba8 [H*W] u32, rgb [H*W][3] f32) of the GPU's render of the
    same view: the subset's oracle pixels are compared with it (max RGBA8
    difference, max RGB error relative to max(|want|, 10 % of the channel's
    RMS), as the parity tests measure them)."""
    from oracle import oracle as orc
    g = orc.make_grid(16, 19, 1)
    table = model.table.numpy().view(np.uint16)
    dp = model.density.numpy().view(np.uint16)
    cp = model.color.numpy().view(np.uint16)
    ocam = orc.camera_from_bytes(bytes(cam))
    b = bits.numpy()
    stride = 4099 * max(1, 16 // threads)
    rays = np.arange(0, W * H, stride, dtype=np.uint32)
    t0 = time.perf_counter()
    orc.render_rays(g, table, dp, cp, ocam, b, 128, (0, 0, 0, 1, 1, 1), MAX_STEPS, rays, T_STOP, threads=threads)
    per_ray = max(time.perf_counter() - t0, 1e-3) / rays.size
    stride = max(1, (W * H) // int(min(W * H, max(rays.size, budget_s / per_ray))))
    rays = np.arange(0, W * H, stride, dtype=np.uint32)
    t0 = time.perf_counter()
    want_rgb, want_rgba, _ = orc.render_rays(g, table, dp, cp, ocam, b, 128, (0, 0, 0, 1, 1, 1), MAX_STEPS, rays, T_STOP, threads=threads)
    dt = time.perf_counter() - t0
    out = {"value": round(rays.size / dt / 1e6, 6), "unit": "Mrays/s", "threads": threads, "seconds": round(dt, 2),
           "sample": f"{rays.size} rays (every {stride}th ray of the {W}x{H} view: full march + field + composite per ray)"}
    if gpu_image is not None:
        g_rgba, g_rgb = gpu_image
        d8 = np.abs(g_rgba[rays].view(np.uint8).astype(int) - want_rgba.view(np.uint8).astype(int)).max()
        wr = want_rgb.astype(np.float64)
        floor = np.maximum(0.1 * np.sqrt(np.mean(wr ** 2, axis=0)), 1e-6)
        rel = (np.abs(g_rgb[rays].astype(np.float64) - wr) / np.maximum(np.abs(wr), floor)).max()
        out["parity_vs_gpu"] = {"rays": int(rays.size), "max_rgba8_diff": int(d8), "max_rgb_rel_err": float(f"{rel:.3e}")}
    return out


def cpu_c1_leg(threads: int):
    """C1 on the oracle: hash encode + density MLP of all 2^16 points (fp32
    table T = 2^16, the parity tests' points and weights)."""
    from nerf_amd import _lib as L, ext
    from oracle import oracle as orc
    n = 1 << 16
    desc = ext.grid_desc(16, L.NERF_EXT_F32)
    table = ext.init_table(desc, 0, 1e-4).numpy()
    dp = ext.mlp_init(0).astype(np.float16).view(np.uint16)
    pos = unit_points(n, seed=0)
    g = orc.make_grid(16, 16, 0)
    t0 = time.perf_counter()
    _threaded(lambda b, e: orc.density_forward(g, table, dp, pos[b:e]), n, threads)
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 1), "unit": "points/s", "threads": threads, "seconds": round(dt, 3), "sample": "all 2^16 points of C1 (hash encode 16 x 2^16 fp32 + density MLP 32-64-16)"}


def cpu_train_leg(snap, threads: int, ray_fraction: float = 1.0):
    """One C3 training step on the oracle, fed the GPU trainer's own inputs
    (camera image, occupancy, model, step index and ray count of a 2^18-sample
    step): march (one thread: the per-ray seeds make it serial here), field
    forward, Huber composite backward per ray, MLP backward, hash-grid
    scatter-add, Adam over the 16.8 M parameters."""
    from oracle import oracle as orc
    n_rays = max(1, int(snap["rays"] * ray_fraction))
    box = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
    times = {}
    t0 = time.perf_counter()
    cap = 1 << 18  # the GPU step's sample capacity: rays past it are cut whole
    counts, gt, pix, offs, tdt = orc.train_rays(snap["ocam"], snap["image"], snap["bits"], 128, box, MAX_STEPS, snap["frame"], n_rays, cap)
    counts = np.where(offs.astype(np.int64) + counts <= cap, counts, 0).astype(np.uint32)
    n = int((offs.astype(np.int64) + counts)[counts > 0].max()) if (counts > 0).any() else 0
    times["march"] = time.perf_counter() - t0
    # Sample positions and directions (host numpy, like the GPU's o + t d).
    c2w = np.array(snap["cam"].c2w[:], np.float32).reshape(3, 4)
    cam = snap["cam"]
    px, py = pix[:, 0], np.float32(cam.height) - np.float32(1.0) - pix[:, 1]
    dcam = np.stack([(px - cam.cx) / cam.fx, (py - cam.cy) / cam.fy, -np.ones_like(px)], 1).astype(np.float32)
    d = dcam @ c2w[:, :3].T
    d = (d / np.linalg.norm(d, axis=1, keepdims=True)).astype(np.float32)
    ray_of = np.repeat(np.arange(n_rays), counts)
    dirs = np.ascontiguousarray(d[ray_of])
    pos = np.clip(c2w[:, 3][None, :] + tdt[:n, 0:1] * dirs, 0.0, 1.0).astype(np.float32)
    g, table, dp, cp = snap["grid"], snap["table"], snap["dp"], snap["cp"]
    t0 = time.perf_counter()
    field = np.concatenate(_threaded(lambda b, e: orc.field_forward(g, table, dp, cp, pos[b:e], dirs[b:e]), n, threads))
    times["forward"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    draw = np.zeros((n, 4), np.float32)
    inv = 1.0 / max(1, int((counts > 0).sum()))

    def comp(rb, re):
        for r in range(rb, re):
            a, c = int(offs[r]), int(counts[r])
            if c:
                _, d1, d3, _ = orc.composite_backward_act(field[a:a + c, 0], field[a:a + c, 1:], tdt[a:a + c, 1], gt[r, :3], delta=0.1, inv_norm=inv)
                draw[a:a + c, 0], draw[a:a + c, 1:] = d1, d3

    _threaded(comp, n_rays, threads)
    times["composite"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    feats = np.concatenate(_threaded(lambda b, e: orc.encode(g, table, pos[b:e]), n, threads))
    parts = _threaded(lambda b, e: orc.mlp_backward(dp, cp, feats[b:e], dirs[b:e], draw[b:e, 0], draw[b:e, 1:], 128.0), n, threads)
    dfeat = np.concatenate([p[0] for p in parts])
    tg = None
    for part in _threaded(lambda b, e: orc.encode_backward(g, pos[b:e], dfeat[b:e]), n, min(threads, 8)):
        tg = part if tg is None else tg + part
    times["backward"] = time.perf_counter() - t0
    t0 = time.perf_counter()
    w = snap["table32"].copy()
    m, v = np.zeros_like(w), np.zeros_like(w)
    orc.adam(w, m, v, tg.astype(np.float32), 1e-2, 0.9, 0.99, 1e-15, 1e30, 1e30, 128.0, 0, 1, 1.0)
    times["adam"] = time.perf_counter() - t0
    total = sum(times.values())
    return {"value": round(n / total, 1), "unit": "train samples/s", "threads": threads, "seconds": round(total, 2), "stage_seconds": {k: round(t, 3) for k, t in times.items()},
            "sample": f"one training step: {int((counts > 0).sum())} rays with samples of {n_rays} marched ({n} samples, capacity 2^18) of the GPU trainer's step {snap['frame']} on the 800x800 camera it picked"
                      + ("" if ray_fraction == 1.0 else f" (the first {ray_fraction:.3g} of its rays)")}


def cpu_baseline(model, cam, bits, train_snap, gpu_image=None):
    """The scalar C++ oracle (the same math, -O2 -ffp-contract=off, no SIMD
    intrinsics) on the host: 1 thread and the host's thread share."""
    threads = min(16, os.cpu_count() or 1)
    legs = {"render_1t": cpu_render_leg(model, cam, bits, 1, 6.0), f"render_{threads}t": cpu_render_leg(model, cam, bits, threads, 6.0, gpu_image), "c1_1t": cpu_c1_leg(1), f"c1_{threads}t": cpu_c1_leg(threads)}
    if train_snap is not None:
        legs["train_1t"] = cpu_train_leg(train_snap, 1, ray_fraction=1.0 / 16)
        legs[f"train_{threads}t"] = cpu_train_leg(train_snap, threads)
    head = legs[f"render_{threads}t"]
    return {"value": head["value"], "unit": "Mrays/s", "cores": threads, "kind": "port", "sample": head["sample"], "parity_vs_gpu": head.get("parity_vs_gpu"), "hardware_concurrency": os.cpu_count(), "cpu_model": _cpu_model(),
            "threads_note": "the host's share of one GPU box is 16 threads (the all-threads legs use them); 1-thread legs alongside", "legs": legs}


def main() -> int:
    global W, H
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-stage-rooflines", action="store_true", help="skip the encode / MLP stage measurements")
    ap.add_argument("--no-configs", action="store_true", help="skip the C4 (1920x1080, T=2^22) and C5 (8 views, 5 cascades) renders")
    ap.add_argument("--train-steps", type=int, default=100, help="timed training steps (0: skip the training leg)")
    ap.add_argument("--train-warmup", type=int, default=30)
    ap.add_argument("--no-reference-legs", action="store_true", help="skip the reference-model training, reference-host and reference-model render legs")
    ap.add_argument("--width", type=int, default=W, help="render width (the metric is quoted at 800)")
    ap.add_argument("--height", type=int, default=H, help="render height (the metric is quoted at 800)")
    ap.add_argument("--only", choices=["render", "stages", "train", "reftrain", "refhost", "configs", "refrender"], default=None,
                    help="run one leg only and print its result (for profiling a leg under rocprofv3): the headline render (3 renders), the stage rooflines, "
                         "training (30 + 30 steps), reference-model training, the reference host's workload, the C4/C5 renders, the reference-model render")
    ap.add_argument("--refhost-steps", type=int, default=60, help="timed steps of the reference-host leg with --only refhost (the full run times 200 in a child process)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain fp32->fp16 conversion over MIB MiB of input (reads 4 B, writes 2 B per element) to calibrate HBM counters, then exit")
    args = ap.parse_args()
    W, H = args.width, args.height
    if args.gpus != 1:
        print(f"bench.py: this backend runs on one GPU; --gpus {args.gpus} is not supported (multi-GPU sharding is design-only)", file=sys.stderr)
        return 2

    from nerf_amd import _lib as L, ext
    from nerf_amd.device import DeviceArray, Event, Stream, device_info, synchronize

    L.load()
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        src, dst = DeviceArray((n,), np.float32), DeviceArray((n,), np.float16)
        src.fill_bytes(0)
        for _ in range(3):
            L.call("nerf_ext_float_to_half", src.ptr, dst.ptr, n, None)
        synchronize()
        print(json.dumps({"copy_calibration": {"elements": n, "read_bytes": 4 * n, "write_bytes": 2 * n, "kernel": "k_float_to_half", "launches": 3}}), flush=True)
        return 0
    if args.only:
        if args.only == "render":
            scene, bits, desc, model, cam, occ = build_workload()
            renderer = ext.Renderer()
            for _ in range(3):
                renderer.render(model, occ, [cam], MAX_STEPS, T_STOP)
            synchronize()
            result = {"renders": 3}
        elif args.only == "stages":
            result = kernel_rooflines(reps_small=50)
        elif args.only == "train":
            result, _ = train_bench(30, 30)
        elif args.only == "reftrain":
            result = ref_train_bench(20, 10)
        elif args.only == "refhost":
            result = reference_host_bench(steps=args.refhost_steps)
        elif args.only == "configs":
            result = config_renders(reps=1)
        else:
            result = ref_model_render(reps=1)
        print(json.dumps({"leg": args.only, "result": result}), flush=True)
        return 0
    t_start = time.perf_counter()

    def progress(what):
        # One stderr line per finished leg (stdout keeps the single JSON line).
        print(f"bench.py: {what} done at {time.perf_counter() - t_start:.1f} s", file=sys.stderr, flush=True)

    info = device_info()
    scene, bits, desc, model, cam, occ = build_workload()
    progress("workload")
    stream = Stream()
    renderer = ext.Renderer()
    rgba = DeviceArray((1, H, W), np.uint32)
    for _ in range(args.warmup):
        renderer.render(model, occ, [cam], MAX_STEPS, T_STOP, rgba8=rgba, stream=stream)
    synchronize()

    # Timed region: K renders back to back on one stream.
    ev0, ev1 = Event(), Event()
    synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        renderer.render(model, occ, [cam], MAX_STEPS, T_STOP, rgba8=rgba, stream=stream)
    ev1.record(stream)
    synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_ms(ev1) / args.steps
    ms_per_step = wall * 1000.0 / args.steps

    # Per-stage timing (HIP events on the render stream) over a second pass.
    stage = {"count": 0.0, "scan": 0.0, "samples": 0.0, "field": 0.0, "composite": 0.0, "total": 0.0}
    samples = 0
    for _ in range(args.steps):
        _, st = renderer.render(model, occ, [cam], MAX_STEPS, T_STOP, rgba8=rgba, stream=stream, timed=True)
        stage["count"] += st.ms_count
        stage["scan"] += st.ms_scan
        stage["samples"] += st.ms_samples
        stage["field"] += st.ms_field
        stage["composite"] += st.ms_composite
        stage["total"] += st.ms_total
        samples = st.samples
        shaded = st.samples_shaded
    stage = {k: v / args.steps for k, v in stage.items()}
    # The image of one more render, with its unclamped RGB, for the CPU leg's
    # parity check (outside the timed region).
    rgb_img = DeviceArray((1, H, W, 3), np.float32)
    renderer.render(model, occ, [cam], MAX_STEPS, T_STOP, rgba8=rgba, rgb=rgb_img, stream=stream)
    synchronize()
    gpu_image = (rgba.numpy().reshape(-1), rgb_img.numpy().reshape(-1, 3))
    del rgb_img
    progress("render")
    field_s = stage["field"] / 1e3
    achieved_gbs = shaded * FIELD_BYTES_PER_SAMPLE / field_s / 1e9
    field_tflops = shaded * FIELD_FLOPS_PER_SAMPLE / field_s / 1e12

    rays = W * H
    line = {
        "metric": "Mrays/s (800x800 render) + train samples/s; % of HBM / MFMA roofline",
        "value": round(rays / (ms_per_step / 1e3) / 1e6, 3),
        "unit": "Mrays/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 MFMA (fp32 accumulate), f32 march/composite",
        "data": "synthetic: analytic 32-Gaussian scene, random-init hash grid and MLPs",
        "config": {"workload": f"{W}x{H} inference render, 32-Gaussian scene, 128^3 occupancy, hash grid T=2^19 fp16, <=1024 steps/ray, early stop T<1e-4",
                   "rays": rays, "samples_per_render": int(samples), "samples_shaded": int(shaded), "gpu_ms_per_render": round(gpu_ms, 4), "parallelism": "single GPU"},
        "stages_ms": {k: round(v, 4) for k, v in stage.items()},
        "roofline": {"kernel": "k_field_forward_lv (fused hash encode + density/colour MLP, level-major gathers)", "bound": "hbm", "achieved": round(achieved_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved_gbs / HBM_PEAK_GBS, 4), "traffic": int(shaded * FIELD_TRAFFIC_BYTES_PER_SAMPLE),
                     "traffic_source": f"profile-derived, not counted in this run: {FIELD_TRAFFIC_BYTES_PER_SAMPLE} B/sample from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE on this render (profiles/field_forward_800x800_counters.md) x this run's shaded samples",
                     "traffic_GBps": round(shaded * FIELD_TRAFFIC_BYTES_PER_SAMPLE / field_s / 1e9, 1), "mfma_tflops": round(field_tflops, 2), "mfma_frac": round(field_tflops / MFMA_FP16_PEAK_TFS, 4),
                     "bytes_per_sample": FIELD_BYTES_PER_SAMPLE, "flops_per_sample": FIELD_FLOPS_PER_SAMPLE},
        "device": {"name": info.name.decode(), "arch": info.arch.decode(), "cus": info.compute_units},
    }
    if not args.no_stage_rooflines:
        line["stage_rooflines"] = kernel_rooflines()
        progress("stage rooflines")
        line["abi_render"] = abi_render()
        progress("ABI render")
    train_snap = None
    if args.train_steps > 0:
        line["train"], train_snap = train_bench(args.train_steps, args.train_warmup)
        progress("training")
        if not args.no_reference_legs:
            line["train_reference_model"] = ref_train_bench(max(10, args.train_steps // 2), 10)
            progress("reference-model training")
            line["reference_host"] = leg_in_child("refhost", ["--refhost-steps", "200"])
            progress("reference host")
    if not args.no_configs:
        line["configs"] = config_renders()
        progress("C4/C5 renders")
        if not args.no_reference_legs:
            line["reference_model"] = ref_model_render()
            progress("reference-model render")
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(model, cam, bits, train_snap, gpu_image)
        progress("CPU baseline")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
