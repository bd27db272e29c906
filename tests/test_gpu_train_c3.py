"""The training configuration of the benchmark (C3) under the oracle.

800x800 views of the 32-Gaussian analytic scene from the orbit at radius 4
(1.32 in the normalised frame), focal 1111 px, hash table T = 2^19 fp16,
up to 1024 march steps per ray, and an adaptive ray count aimed at a sample
target.  At this focal length the cone step is below the minimum step for
most of a ray, so rays take several hundred steps: the training sampler's
emission pass resumes 64-step segments from the checkpoints of its count
pass (backend-cuda.cu:422-533 restated as one serial march in the oracle),
and these tests hold that resume path to the oracle bit for bit.

Bars: per-ray counts, offsets, kept counts, (t_mid, dt) and owning rays
bit-exact; the ray count of every step equal to the controller's fp32
recurrence; features, field outputs and composite gradients within 1e-3
relative; weight and table gradients within 1e-2 relative (Frobenius);
Adam (clip 1, guard 100, decay 250 k steps, the reference host's settings,
backend-cuda.cu:1513-1554) within 1e-5 of the oracle on the GPU's own
gradients.
"""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, oracle_grid, assert_rel, assert_adam_step, assert_table_grad, assert_rel_rows, fixed_point_floor

pytestmark = pytest.mark.gpu

W = H = 800
FOCAL = 1111.0
VIEWS = 8
CENTRE = (0.5, 0.5, 0.5)
BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
OCC_RES = 128
STEPS = 1024
LOG2_T = 19
LOSS_SCALE = 128.0
SEG = 64  # march steps per resumable segment of the training sampler


@pytest.fixture(scope="module")
def scene():
    g = ext.scene_gaussians(32, seed=11)
    cams = [ext.camera_orbit(17, i, 1.32, CENTRE, W, H, FOCAL) for i in range(VIEWS)]
    imgs = ext.scene_render(g, cams, 256).numpy()
    bits = orc.occupancy_from_scene(g, OCC_RES, threshold=0.01)
    assert 0.05 < np.unpackbits(bits.view(np.uint8)).mean() < 0.95, "scene occupancy neither empty nor full"
    return g, cams, imgs, bits


def _trainer(scene, *, target, initial_rays, max_rays, capacity, hyper=None):
    _, cams, imgs, _ = scene
    grid = ext.grid_desc(LOG2_T, L.NERF_EXT_F16)
    occ = ext.occupancy_params(warmup_steps=256, update_interval=16, cells_per_update=65536, threshold=0.01, decay=0.95)
    hyper = hyper or ext.hyper_params(lr=1e-2, beta1=0.9, beta2=0.99, eps=1e-15, loss_scale=LOSS_SCALE)
    t = ext.Trainer(grid, imgs.view(np.uint8), cams, occupancy_res=OCC_RES, hyper=hyper, occupancy=occ, initial_rays=initial_rays, max_rays=max_rays, target_samples=target, sample_capacity=capacity,
                    max_steps_per_ray=STEPS, seed=7, table_init_range=1e-1)
    return t, grid


def _run_steps_checking_controller(t, steps, target, initial_rays, max_rays):
    """Runs whole steps one at a time; every step's ray count must follow the
    device controller's fp32 recurrence (half-way towards the ray count that
    would have hit the target with the step's occupied samples before the
    capacity cut, clamped to [64, max_rays])."""
    rf = np.float32(initial_rays)
    seen = []
    for k in range(steps):
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_END)
        st = t.stats()
        want_rays = min(max(int(np.float32(rf + np.float32(0.5))), 64), max_rays)
        assert st.rays == want_rays, f"step {k}: {st.rays} rays, controller recurrence gives {want_rays}"
        assert st.last.has_nonfinite == 0
        n = st.occupied_samples
        if n > 0:
            want = np.float32(np.float32(rf * np.float32(target)) / np.float32(n))
            rf = np.float32(np.float32(np.float32(0.5) * rf) + np.float32(np.float32(0.5) * want))
            rf = np.float32(min(max(rf, np.float32(64.0)), np.float32(max_rays)))
        seen.append((st.rays, st.samples, n))
    return seen, rf


def _load_scene_bits(t, bits):
    """Replaces the trainer's occupancy (all ones during warmup) by the
    scene's, so that rays hold occupied runs separated by empty space.  The
    copy runs on the null stream: the trainer's stream (whose warmup kernel
    writes the bits) is drained first."""
    t.synchronize()
    ext.write_device(t.buffers().bitfield, bits)


def _sample_state(t, n_rays):
    B = t.buffers()
    st = t.stats()
    n = st.samples
    return dict(
        stats=st,
        counts=ext.read_device(B.counts, (n_rays,), np.uint32),
        kept=ext.read_device(B.kept, (n_rays,), np.uint32),
        offsets=ext.read_device(B.offsets, (n_rays,), np.uint32),
        gt=ext.read_device(B.gt, (n_rays, 4), np.float32),
        rays=ext.read_device(B.rays, (n_rays, 2, 4), np.float32),
        samples=ext.read_device(B.samples, (n, 2), np.float32),
        sample_ray=ext.read_device(B.sample_ray, (n,), np.uint32),
    )


def _check_sample_stage(s, scene, frame, capacity):
    _, cams, imgs, bits = scene
    n_rays = s["stats"].rays
    cam = orc.train_camera(frame, VIEWS)
    counts, gt, _, offs, tdt = orc.train_rays(orc.camera_from_bytes(bytes(cams[cam])), imgs[cam].view(np.uint8), bits, OCC_RES, BOX, STEPS, frame, n_rays, capacity)
    assert np.array_equal(s["counts"], counts), "per-ray occupied-step counts"
    assert np.array_equal(s["offsets"], offs), "per-ray offsets"
    hit = counts > 0
    np.testing.assert_allclose(s["gt"][hit], gt[hit], rtol=0, atol=1e-6)
    fits = hit & (offs.astype(np.int64) + counts <= capacity)
    assert np.array_equal(s["kept"], np.where(fits, counts, 0)), "kept counts"
    n = int((offs.astype(np.int64) + counts)[fits].max()) if fits.any() else 0
    assert s["stats"].samples == n
    assert s["stats"].active_rays == int(fits.sum())
    assert np.array_equal(s["samples"].view(np.uint32), tdt[:n].view(np.uint32)), "(t_mid, dt) of the kept samples"
    assert np.array_equal(s["sample_ray"], np.repeat(np.arange(n_rays, dtype=np.uint32)[fits], counts[fits])), "owning ray of each sample"
    # The resume path is exercised: with every cell occupied the same rays
    # take this many steps (the segment structure depends on steps, not on
    # occupied samples).
    all_steps, *_ = orc.train_rays(orc.camera_from_bytes(bytes(cams[cam])), imgs[cam].view(np.uint8), np.full_like(bits, 0xFFFFFFFF), OCC_RES, BOX, STEPS, frame, n_rays, 1)
    return counts, offs, all_steps


@pytest.fixture(scope="module")
def c3_step(scene):
    """Three adaptive steps (target 2^16 samples), then step 3 stage by stage
    on the scene's occupancy, with host snapshots after each stage."""
    target, init, max_rays, cap = 1 << 16, 256, 1 << 15, 1 << 17
    t, grid = _trainer(scene, target=target, initial_rays=init, max_rays=max_rays, capacity=cap)
    seen, _ = _run_steps_checking_controller(t, 3, target, init, max_rays)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
    _load_scene_bits(t, scene[3])
    t.run_stages(L.NERF_EXT_STAGE_SAMPLE, L.NERF_EXT_STAGE_SAMPLE)
    n_rays = t.stats().rays
    s = _sample_state(t, n_rays)
    m, _ = t.model()
    B = t.buffers()
    table = ext.read_device(m.table, (int(B.table_elems),), np.uint16)
    dp = ext.read_device(m.density_params, (L.NERF_EXT_DENSITY_PARAMS,), np.uint16)
    cp = ext.read_device(m.color_params, (L.NERF_EXT_COLOR_PARAMS,), np.uint16)
    t.run_stages(L.NERF_EXT_STAGE_FORWARD, L.NERF_EXT_STAGE_BACKWARD)
    t.synchronize()  # the trainer's stream does not order with the copies below
    n = s["stats"].samples
    assert not B.features_lm, "1,024 steps per ray keep the features as rows"
    out = dict(trainer=t, grid=grid, seen=seen, s=s, table=table, dp=dp, cp=cp, cap=cap,
               field=ext.read_device(B.field, (n, 4), np.float32),
               features=ext.read_device(B.features, (n, 32), np.float16).astype(np.float32),
               draw=ext.read_device(B.draw, (n, 4), np.float32),
               mlp_grad=ext.read_device(B.mlp_grad, (10240,), np.float32),
               table_grad=ext.read_device(B.table_grad, (int(B.table_elems),), np.float32),
               dfeat=ext.read_device(B.dfeat, (16, int(B.sample_capacity), 2), np.float32)[:, :n, :].transpose(1, 0, 2).reshape(n, 32))
    return out


def _positions(s):
    r = s["sample_ray"]
    ro, rd = s["rays"][r, 0], s["rays"][r, 1]
    w = ro[:, :3] + s["samples"][:, 0:1] * rd[:, :3]
    return w.astype(np.float32), np.ascontiguousarray(rd[:, :3])


def test_controller_adapts(c3_step):
    announce("C3 controller: ray count over three steps")
    seen = c3_step["seen"]
    assert seen[0][0] == 256
    assert seen[2][0] != seen[0][0], f"the ray count did not adapt: {seen}"


def test_sample_stage_multi_segment(c3_step, scene):
    announce("C3 sample stage, 1024 steps/ray, scene occupancy, frame 3")
    s = c3_step["s"]
    counts, _, all_steps = _check_sample_stage(s, scene, 3, c3_step["cap"])
    assert s["stats"].samples > 20000, "too few samples for a C3-sized check"
    assert (all_steps > 3 * SEG).mean() > 0.5, "most rays must span more than three 64-step segments"
    assert all_steps.max() > 10 * SEG
    assert (counts > 0).mean() > 0.2


def test_forward_stage(c3_step):
    announce("C3 forward stage (T=2^19)")
    s, og = c3_step["s"], oracle_grid(c3_step["grid"])
    p, d = _positions(s)
    want_feat = orc.encode(og, c3_step["table"], p)
    assert_rel(c3_step["features"], want_feat, what="training features (fp16)")
    want = orc.field_forward(og, c3_step["table"], c3_step["dp"], c3_step["cp"], p, d)
    assert_rel(c3_step["field"][:, 0], want[:, 0], what="sigma", mlp=True)
    assert_rel(c3_step["field"][:, 1:], want[:, 1:], what="rgb", mlp=True)


def _composite_oracle(s, field, inv_norm):
    n = s["stats"].samples
    ds = np.zeros(n, np.float32)
    drgb = np.zeros((n, 3), np.float32)
    for r in np.nonzero(s["kept"])[0]:
        b, c = int(s["offsets"][r]), int(s["kept"][r])
        sl = slice(b, b + c)
        _, d1, d3, _ = orc.composite_backward_act(field[sl, 0], field[sl, 1:], s["samples"][sl, 1], s["gt"][r, :3], delta=0.1, inv_norm=inv_norm)
        ds[sl], drgb[sl] = d1, d3
    return ds, drgb


def test_composite_stage(c3_step):
    announce("C3 composite stage")
    s = c3_step["s"]
    ds, drgb = _composite_oracle(s, c3_step["field"], 1.0 / s["stats"].active_rays)
    assert_rel(c3_step["draw"][:, 0], ds, what="d sigma_raw")
    assert_rel(c3_step["draw"][:, 1:], drgb, what="d rgb_raw")


def _frob(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def test_backward_stage(c3_step):
    announce("C3 backward stage (T=2^19)")
    s = c3_step["s"]
    p, d = _positions(s)
    draw = c3_step["draw"]
    dfeat, dD, dC = orc.mlp_backward(c3_step["dp"], c3_step["cp"], c3_step["features"], d, draw[:, 0], draw[:, 1:], LOSS_SCALE)
    g = c3_step["mlp_grad"]
    assert np.isfinite(g).all() and np.isfinite(c3_step["table_grad"]).all()
    for name, got, want in (("density input", g[:2048], dD[:2048]), ("density output", g[2048:3072], dD[2048:]), ("colour input", g[3072:5120], dC[:2048]),
                            ("colour hidden", g[5120:9216], dC[2048:6144]), ("colour output", g[9216:], dC[6144:])):
        err = _frob(got, want)
        print(f"[grad] C3 {name} dW: relative Frobenius {err:.3e}", flush=True)
        assert err < 1e-3, f"{name} dW: relative Frobenius error {err:.3e}"
    assert_rel_rows(c3_step["dfeat"], dfeat, what="C3 d features")
    og = oracle_grid(c3_step["grid"])
    floor = fixed_point_floor(c3_step["dfeat"])
    assert_table_grad(c3_step["table_grad"], orc.encode_backward(og, p, c3_step["dfeat"]), 16, "C3 table gradient (scatter)", frob_tol=1e-3, floor=floor)
    # End to end: the samples whose ReLU mask flipped move the few entries they touch.
    assert_table_grad(c3_step["table_grad"], orc.encode_backward(og, p, dfeat), 16, "C3 table gradient (end to end)", frob_tol=1e-3, floor=floor, entry_frac=1e-4)


def test_adam_reference_settings(scene):
    """Three steps with clip 1, guard 100 and lr decay over 250 k steps (the
    reference host's hyper-parameters); each step's update against the
    oracle's Adam on the GPU's own gradients."""
    announce("C3 Adam, clip 1 / guard 100 / decay 250")
    hyper = ext.hyper_params(lr=1e-2, beta1=0.9, beta2=0.99, eps=1e-15, clip=1.0, guard=100.0, loss_scale=LOSS_SCALE, lr_decay_ksteps=250)
    t, _ = _trainer(scene, target=1 << 15, initial_rays=256, max_rays=1 << 14, capacity=1 << 16, hyper=hyper)
    B = t.buffers()
    E = int(B.table_elems)
    for step in range(3):
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
        t.synchronize()
        state = {k: ext.read_device(getattr(B, k), (E if k.startswith("table") else 10240,), np.float32) for k in ("table_f32", "table_m", "table_v", "table_grad", "mlp_f32", "mlp_m", "mlp_v", "mlp_grad")}
        gn = float(np.sqrt(np.sum(state["table_grad"].astype(np.float64) ** 2) + np.sum(state["mlp_grad"].astype(np.float64) ** 2))) / LOSS_SCALE
        t.run_stages(L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)
        st = t.stats()
        assert st.skipped == 0 and st.last.has_nonfinite == 0
        assert abs(st.last.grad_norm - gn) <= 1e-4 * gn
        for part in ("table", "mlp"):
            w, m, v = state[f"{part}_f32"].copy(), state[f"{part}_m"].copy(), state[f"{part}_v"].copy()
            skipped = orc.adam(w, m, v, state[f"{part}_grad"], 1e-2, 0.9, 0.99, 1e-15, 1.0, 100.0, LOSS_SCALE, 250, step + 1, gn)
            assert skipped == 0
            got_w = ext.read_device(getattr(B, f"{part}_f32"), w.shape, np.float32)
            got_m = ext.read_device(getattr(B, f"{part}_m"), w.shape, np.float32)
            assert_adam_step(got_w, state[f"{part}_f32"], w, what=f"step {step}: {part} Adam update")
            np.testing.assert_allclose(got_m, m, rtol=1e-5, atol=1e-6 * float(np.abs(m).max()), err_msg=f"step {step}: {part} first moment")


def test_c3_target_2p18(scene):
    """The benchmark's batch: 2^18 samples per step.  Four adaptive steps
    starting from 1,024 rays, then the fifth step's sample stream on the
    scene's occupancy, bit-exact."""
    announce("C3 sampler at the 2^18-sample target")
    target, init, max_rays, cap = 1 << 18, 1024, 1 << 16, 1 << 19
    t, _ = _trainer(scene, target=target, initial_rays=init, max_rays=max_rays, capacity=cap)
    seen, _ = _run_steps_checking_controller(t, 4, target, init, max_rays)
    assert abs(seen[-1][2] - target) < 0.5 * target, f"controller far from the target: {seen}"
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
    _load_scene_bits(t, scene[3])
    t.run_stages(L.NERF_EXT_STAGE_SAMPLE, L.NERF_EXT_STAGE_SAMPLE)
    s = _sample_state(t, t.stats().rays)
    _check_sample_stage(s, scene, 4, cap)


def test_capacity_cut_mid_segment(scene):
    """A stream capacity that ends inside a long ray's sample range, past its
    first segment: that ray and every later one are dropped whole, the rays
    before it are kept bit-exact."""
    announce("C3 sampler, capacity cut inside a multi-segment ray")
    _, cams, imgs, bits = scene
    rays = 2048
    cam = orc.train_camera(0, VIEWS)
    counts, _, _, offs, _ = orc.train_rays(orc.camera_from_bytes(bytes(cams[cam])), imgs[cam].view(np.uint8), bits, OCC_RES, BOX, STEPS, 0, rays, 1)
    all_steps, *_ = orc.train_rays(orc.camera_from_bytes(bytes(cams[cam])), imgs[cam].view(np.uint8), np.full_like(bits, 0xFFFFFFFF), OCC_RES, BOX, STEPS, 0, rays, 1)
    long_rays = np.nonzero((counts > 2 * SEG) & (all_steps > 4 * SEG) & (np.arange(rays) > rays // 4))[0]
    assert long_rays.size, "no ray with occupied samples over several segments"
    r = int(long_rays[0])
    cap = int(offs[r]) + int(counts[r]) // 2
    t, _ = _trainer(scene, target=0, initial_rays=rays, max_rays=rays, capacity=cap)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
    _load_scene_bits(t, bits)
    t.run_stages(L.NERF_EXT_STAGE_SAMPLE, L.NERF_EXT_STAGE_SAMPLE)
    s = _sample_state(t, rays)
    _check_sample_stage(s, scene, 0, cap)
    assert s["kept"][r] == 0 and s["kept"][:r][counts[:r] > 0].all()
