"""GPU training-step parity, stage by stage, against the oracle.

Bars: sample counts, offsets and (t_mid, dt) bit-exact; ground truth within
1e-6; field outputs, composite gradients and the loss within 1e-3 relative;
MLP weight gradients and hash-table gradients within 1e-2 relative (Frobenius
norm; fp16 ReLU masks may flip on a few activations); Adam within 1e-5 on the
GPU's own gradients.  The dataset is the analytic Gaussian scene rendered by
nerf_ext_scene_render (itself checked against the oracle to 1 LSB).
"""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, oracle_grid, assert_rel, assert_adam_step, assert_table_grad, assert_rel_rows, fixed_point_floor

pytestmark = pytest.mark.gpu

W = H = 64
VIEWS = 4
FOCAL = 1111.0 * W / 800.0
CENTRE = (0.5, 0.5, 0.5)
BOX = (0.0, 0.0, 0.0, 1.0, 1.0, 1.0)
OCC_RES = 32
RAYS = 256
STEPS = 64
LOSS_SCALE = 128.0


@pytest.fixture(scope="module")
def dataset():
    g = ext.scene_gaussians(16, seed=3)
    cams = [ext.camera_orbit(7, i, 1.32, CENTRE, W, H, FOCAL) for i in range(VIEWS)]
    imgs = ext.scene_render(g, cams, 128).numpy()
    return g, cams, imgs


def _trainer(dataset, capacity=RAYS * STEPS, rays=RAYS, log2_table=14, hyper=None, occ=None, max_rays=None, **kw):
    _, cams, imgs = dataset
    grid = ext.grid_desc(log2_table, L.NERF_EXT_F16)
    occ = occ or ext.occupancy_params(warmup_steps=2, update_interval=4, cells_per_update=OCC_RES ** 3, threshold=0.01, decay=0.95)
    hyper = hyper or ext.hyper_params(loss_scale=LOSS_SCALE)
    t = ext.Trainer(grid, imgs.view(np.uint8), cams, occupancy_res=OCC_RES, hyper=hyper, occupancy=occ, initial_rays=rays, max_rays=max_rays or rays, sample_capacity=capacity, max_steps_per_ray=STEPS,
                    seed=5, table_init_range=1e-1, **kw)
    return t, grid


def _model_host(t):
    m, _ = t.model()
    elems = ext.table_elements(m.grid)
    table = ext.read_device(m.table, (elems,), np.uint16)
    dp = ext.read_device(m.density_params, (L.NERF_EXT_DENSITY_PARAMS,), np.uint16)
    cp = ext.read_device(m.color_params, (L.NERF_EXT_COLOR_PARAMS,), np.uint16)
    return table, dp, cp


def _sample_state(t):
    """Device buffers after the SAMPLE stage, as host arrays."""
    B = t.buffers()
    st = t.stats()
    n = st.samples
    return dict(
        stats=st,
        counts=ext.read_device(B.counts, (RAYS,), np.uint32),
        kept=ext.read_device(B.kept, (RAYS,), np.uint32),
        offsets=ext.read_device(B.offsets, (RAYS,), np.uint32),
        gt=ext.read_device(B.gt, (RAYS, 4), np.float32),
        rays=ext.read_device(B.rays, (RAYS, 2, 4), np.float32),
        samples=ext.read_device(B.samples, (n, 2), np.float32),
        sample_ray=ext.read_device(B.sample_ray, (n,), np.uint32),
    )


def _features(t, n):
    """The step's fp16 features [n][32]: rows, or the level-major pairs that
    batches of at most 128 steps per ray keep instead."""
    B = t.buffers()
    if B.features_lm:
        lm = ext.read_device(B.features_lm, (16, B.sample_capacity), np.uint32)[:, :n]
        return np.ascontiguousarray(lm.T).view(np.float16).reshape(n, 32).astype(np.float32)
    return ext.read_device(B.features, (n, 32), np.float16).astype(np.float32)


def _positions(s):
    """Normalised sample positions and directions, in the fp32 order the field kernel uses."""
    r = s["sample_ray"]
    ro, rd = s["rays"][r, 0], s["rays"][r, 1]
    t = s["samples"][:, 0:1]
    w = ro[:, :3] + t * rd[:, :3]
    box_min, box_max = np.array(BOX[:3], np.float32), np.array(BOX[3:], np.float32)
    p = ((w - box_min) / (box_max - box_min)).astype(np.float32)
    return p, np.ascontiguousarray(rd[:, :3])


def test_scene_render_matches_oracle(dataset):
    announce("scene render 4 views 64x64")
    g, cams, imgs = dataset
    for v in range(VIEWS):
        want = orc.scene_render(g, orc.camera_from_bytes(bytes(cams[v])), 128).view(np.uint8).reshape(H, W, 4).astype(int)
        got = imgs[v].view(np.uint8).reshape(H, W, 4).astype(int)
        diff = np.abs(got - want)
        assert diff.max() <= 1, f"view {v}: max diff {diff.max()}"
        assert (diff == 0).mean() > 0.99
        assert (got[..., 3] > 0).mean() > 0.05, "scene not visible"


# The warmup sets every bit whatever the threshold (backend-cuda.cu:1569-1571),
# also one above the warmup density of 1.
@pytest.mark.parametrize("threshold", [0.01, 2.0])
def test_occupancy_warmup_marks_every_cell(dataset, threshold):
    announce(f"train occupancy warmup, threshold {threshold}")
    occ = ext.occupancy_params(warmup_steps=2, update_interval=4, cells_per_update=OCC_RES ** 3, threshold=threshold, decay=0.95)
    t, _ = _trainer(dataset, occ=occ)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
    t.synchronize()
    B = t.buffers()
    cells = OCC_RES ** 3
    assert np.all(ext.read_device(B.density_grid, (cells,), np.float32) == 1.0)
    assert np.all(ext.read_device(B.bitfield, (cells // 32,), np.uint32) == 0xFFFFFFFF)


# "together": the begin stage folded into the ray pass; "one_by_one": each
# stage launched alone (the begin in a kernel of its own); "wide": 2^15 ray
# slots, of which the step uses its 256.
@pytest.mark.parametrize("capacity,mode", [(RAYS * STEPS, "together"), (3000, "together"), (3000, "one_by_one"), (3000, "wide")])
def test_sample_stage_bit_exact(dataset, capacity, mode):
    announce(f"train sample stage capacity={capacity} {mode}")
    _, cams, imgs = dataset
    t, _ = _trainer(dataset, capacity=capacity, max_rays=(1 << 15) if mode == "wide" else None)
    if mode == "one_by_one":
        for s in (L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY, L.NERF_EXT_STAGE_SAMPLE):
            t.run_stages(s, s)
    else:
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_SAMPLE)
    s = _sample_state(t)
    cam = orc.train_camera(0, VIEWS)
    bits = ext.read_device(t.buffers().bitfield, (OCC_RES ** 3 // 32,), np.uint32)
    counts, gt, _, offs, tdt = orc.train_rays(orc.camera_from_bytes(bytes(cams[cam])), imgs[cam].view(np.uint8), bits, OCC_RES, BOX, STEPS, 0, RAYS, RAYS * STEPS)
    assert s["stats"].rays == RAYS
    assert np.array_equal(s["counts"], counts)
    assert np.array_equal(s["offsets"], offs)
    hit = counts > 0
    np.testing.assert_allclose(s["gt"][hit], gt[hit], rtol=0, atol=1e-6)
    # Kept rays: the prefix whose samples fit the capacity.
    fits = hit & (offs.astype(np.int64) + counts <= capacity)
    assert np.array_equal(s["kept"], np.where(fits, counts, 0))
    n = int((offs + counts)[fits].max()) if fits.any() else 0
    assert s["stats"].samples == n
    assert s["stats"].active_rays == int(fits.sum())
    assert np.array_equal(s["samples"].view(np.uint32), tdt[:n].view(np.uint32))
    want_ray = np.repeat(np.arange(RAYS, dtype=np.uint32)[fits], counts[fits])
    assert np.array_equal(s["sample_ray"], want_ray)


@pytest.mark.parametrize("log2_table", [14, 19])
def test_forward_stage(dataset, log2_table):
    """At 64 steps per ray the forward takes the level-split encode and the
    MLP pass: four levels per XCD at T = 2^14, one level per XCD in two
    launches at T = 2^19."""
    announce(f"train forward stage, T=2^{log2_table}")
    t, grid = _trainer(dataset, log2_table=log2_table)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_FORWARD)
    s = _sample_state(t)
    n = s["stats"].samples
    B = t.buffers()
    field = ext.read_device(B.field, (n, 4), np.float32)
    assert B.features_lm, "64 steps per ray keep the features level-major"
    feats = _features(t, n)
    table, dp, cp = _model_host(t)
    p, d = _positions(s)
    og = oracle_grid(grid)
    want_feat = orc.encode(og, table, p)
    assert_rel(feats, want_feat, what="training features (fp16)")
    assert (feats == want_feat.astype(np.float16).astype(np.float32)).mean() > 0.999, "features are not the fp16 rounding of the encoding"
    want = orc.field_forward(og, table, dp, cp, p, d)
    assert_rel(field[:, 0], want[:, 0], what="sigma", mlp=True)
    assert_rel(field[:, 1:], want[:, 1:], what="rgb", mlp=True)


def _composite_oracle(s, field, inv_norm):
    n = s["stats"].samples
    ds = np.zeros(n, np.float32)
    drgb = np.zeros((n, 3), np.float32)
    loss = 0.0
    for r in np.nonzero(s["kept"])[0]:
        b, c = int(s["offsets"][r]), int(s["kept"][r])
        sl = slice(b, b + c)
        l, d1, d3, _ = orc.composite_backward_act(field[sl, 0], field[sl, 1:], s["samples"][sl, 1], s["gt"][r, :3], delta=0.1, inv_norm=inv_norm)
        ds[sl], drgb[sl] = d1, d3
        loss += l
    return loss * inv_norm, ds, drgb


def test_composite_stage(dataset):
    announce("train composite stage")
    t, _ = _trainer(dataset)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_COMPOSITE)
    s = _sample_state(t)
    n = s["stats"].samples
    B = t.buffers()
    field = ext.read_device(B.field, (n, 4), np.float32)
    draw = ext.read_device(B.draw, (n, 4), np.float32)
    _, ds, drgb = _composite_oracle(s, field, 1.0 / s["stats"].active_rays)
    assert_rel(draw[:, 0], ds, what="d sigma_raw")
    assert_rel(draw[:, 1:], drgb, what="d rgb_raw")


def _frob(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


# T = 2^14: the dense levels take the coarse LDS slabs, the hashed ones bins.
# T = 2^17: the coarsest dense levels take the slabs (the largest one two of
# them), the finer dense ones bins as well.
@pytest.mark.parametrize("log2_table", [14, 17])
def test_backward_stage(dataset, log2_table):
    announce(f"train backward stage, T=2^{log2_table}")
    t, grid = _trainer(dataset, log2_table=log2_table)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
    s = _sample_state(t)
    n = s["stats"].samples
    B = t.buffers()
    feats = _features(t, n)
    draw = ext.read_device(B.draw, (n, 4), np.float32)
    mlp_grad = ext.read_device(B.mlp_grad, (10240,), np.float32)
    table_grad = ext.read_device(B.table_grad, (B.table_elems,), np.float32)
    _, dp, cp = _model_host(t)
    p, d = _positions(s)
    dfeat, dD, dC = orc.mlp_backward(dp, cp, feats, d, draw[:, 0], draw[:, 1:], LOSS_SCALE)
    assert np.isfinite(mlp_grad).all() and np.isfinite(table_grad).all()
    for name, got, want in (("density input", mlp_grad[:2048], dD[:2048]), ("density output", mlp_grad[2048:3072], dD[2048:]), ("colour input", mlp_grad[3072:5120], dC[:2048]),
                            ("colour hidden", mlp_grad[5120:9216], dC[2048:6144]), ("colour output", mlp_grad[9216:], dC[6144:])):
        err = _frob(got, want)
        print(f"[grad] {name} dW: relative Frobenius {err:.3e}", flush=True)
        assert err < 1e-3, f"{name} dW: relative Frobenius error {err:.3e}"
    # The MLP's input gradient (fp16 deltas at the oracle's rounding points).
    gpu_dfeat = ext.read_device(B.dfeat, (16, int(B.sample_capacity), 2), np.float32)[:, :n, :].transpose(1, 0, 2).reshape(n, 32)
    assert_rel_rows(gpu_dfeat, dfeat, what="d features")
    og = oracle_grid(grid)
    # The scatter-add alone, on the GPU's own d features: exact fixed-point
    # bins and slabs, 17-bit records.
    floor = fixed_point_floor(gpu_dfeat)
    assert_table_grad(table_grad, orc.encode_backward(og, p, gpu_dfeat), 16, f"table gradient (scatter), T=2^{log2_table}", frob_tol=1e-3, floor=floor)
    # End to end from the oracle's d features: the samples whose ReLU mask
    # flipped (bounded above) move the few entries they touch.
    assert_table_grad(table_grad, orc.encode_backward(og, p, dfeat), 16, f"table gradient (end to end), T=2^{log2_table}", frob_tol=1e-3, floor=floor, entry_frac=1e-4)


@pytest.mark.parametrize("log2_table", [14, 17])
def test_adam_stage_and_step_end(dataset, log2_table):
    announce(f"train adam stage, T=2^{log2_table}")
    t, _ = _trainer(dataset, log2_table=log2_table)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
    t.synchronize()
    B = t.buffers()
    E = int(B.table_elems)
    tw = ext.read_device(B.table_f32, (E,), np.float32)
    tg = ext.read_device(B.table_grad, (E,), np.float32)
    mw = ext.read_device(B.mlp_f32, (10240,), np.float32)
    mg = ext.read_device(B.mlp_grad, (10240,), np.float32)
    s = _sample_state(t)
    field = ext.read_device(B.field, (s["stats"].samples, 4), np.float32)
    want_loss, _, _ = _composite_oracle(s, field, 1.0 / s["stats"].active_rays)
    gn = float(np.sqrt(np.sum(tg.astype(np.float64) ** 2) + np.sum(mg.astype(np.float64) ** 2))) / LOSS_SCALE
    t.run_stages(L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)
    st = t.stats()
    hp = t.desc.hyper
    for name, w0, g, ptr, p16, count in (("table", tw, tg, B.table_f32, t.model()[0].table, E), ("mlp", mw, mg, B.mlp_f32, None, 10240)):
        w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
        skipped = orc.adam(w, m, v, g, hp.learning_rate, hp.adam_beta1, hp.adam_beta2, hp.adam_eps, hp.grad_clip_norm, hp.update_guard_grad_norm, LOSS_SCALE, hp.lr_decay_ksteps, 1, gn)
        assert skipped == 0
        got = ext.read_device(ptr, (count,), np.float32)
        np.testing.assert_allclose(got - w0, w - w0, rtol=1e-5, atol=1e-8, err_msg=f"{name} Adam update")
        if p16 is not None:
            assert np.array_equal(ext.read_device(p16, (count,), np.float16), got.astype(np.float16)), "fp16 working copy != RNE(master)"
    # Adam reads the gradients and leaves them as they are (the next backward overwrites them).
    assert np.array_equal(ext.read_device(B.table_grad, (E,), np.float32), tg)
    assert st.last.completed_steps == 1
    assert st.last.last_train_camera == orc.train_camera(0, VIEWS)
    assert st.last.has_nonfinite == 0
    assert abs(st.last.loss - want_loss) <= 1e-3 * want_loss
    assert abs(st.last.grad_norm - gn) <= 1e-4 * gn


def test_occupancy_refresh(dataset):
    announce("train occupancy refresh at step 4")
    t, grid = _trainer(dataset)
    t.step(4)
    t.synchronize()
    table, dp, _ = _model_host(t)
    B = t.buffers()
    cells = OCC_RES ** 3
    before = ext.read_device(B.density_grid, (cells,), np.float32)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
    t.synchronize()
    got = ext.read_device(B.density_grid, (cells,), np.float32)
    bits = ext.read_device(B.bitfield, (cells // 32,), np.uint32)
    idx = np.arange(cells)
    x, y, z = idx % OCC_RES, (idx // OCC_RES) % OCC_RES, idx // (OCC_RES * OCC_RES)
    step = np.float32(1.0 / OCC_RES)
    centres = np.stack([(x + 0.5) * step, (y + 0.5) * step, (z + 0.5) * step], 1).astype(np.float32)
    sigma = orc.density_forward(oracle_grid(grid), table, dp, centres)[:, 0]
    want = np.maximum(before * np.float32(0.95), sigma)
    assert_rel(got, want, what="density grid after refresh")
    occ = got > 0.01
    want_bits = np.packbits(occ.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").ravel().astype(np.uint32)
    assert np.array_equal(bits, want_bits), "bitfield != density > threshold"


def test_training_reduces_loss(dataset):
    announce("train 300 steps")
    t, _ = _trainer(dataset, rays=RAYS)
    losses = []
    for _ in range(30):
        t.step(10)
        st = t.stats()
        assert st.last.has_nonfinite == 0
        losses.append(st.last.loss)
    assert st.last.completed_steps == 300
    assert np.mean(losses[-5:]) < 0.5 * np.mean(losses[:2]), losses


def _optimizer_state(t):
    B = t.buffers()
    E = int(B.table_elems)
    return {k: ext.read_device(getattr(B, k), (E if k.startswith("table") else 10240,), np.float32) for k in ("table_f32", "table_m", "table_v", "table_grad", "mlp_f32", "mlp_m", "mlp_v", "mlp_grad")}


def _grad_norm(state):
    return float(np.sqrt(np.sum(state["table_grad"].astype(np.float64) ** 2) + np.sum(state["mlp_grad"].astype(np.float64) ** 2))) / LOSS_SCALE


def test_adam_clip_and_decay(dataset):
    """Clip factor active (clip far below the gradient norm), learning-rate
    decay on, three steps with nonzero moments (backend-cuda.cu:1513-1554)."""
    announce("train adam: clip + lr decay, three steps")
    clip, decay = 1e-4, 1
    hyper = ext.hyper_params(clip=clip, guard=1e30, loss_scale=LOSS_SCALE, lr_decay_ksteps=decay)
    t, _ = _trainer(dataset, hyper=hyper)
    B = t.buffers()
    for step in range(3):
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
        t.synchronize()
        state = _optimizer_state(t)
        gn = _grad_norm(state)
        assert gn > 10 * clip, f"the clip branch is not active (norm {gn})"
        t.run_stages(L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)
        st = t.stats()
        assert st.skipped == 0 and st.last.has_nonfinite == 0
        hp = t.desc.hyper
        for part in ("table", "mlp"):
            w, m, v = state[f"{part}_f32"].copy(), state[f"{part}_m"].copy(), state[f"{part}_v"].copy()
            assert orc.adam(w, m, v, state[f"{part}_grad"], hp.learning_rate, hp.adam_beta1, hp.adam_beta2, hp.adam_eps, clip, hp.update_guard_grad_norm, LOSS_SCALE, decay, step + 1, gn) == 0
            got_w = ext.read_device(getattr(B, f"{part}_f32"), w.shape, np.float32)
            assert_adam_step(got_w, state[f"{part}_f32"], w, what=f"step {step}: {part} update")
            np.testing.assert_allclose(ext.read_device(getattr(B, f"{part}_m"), w.shape, np.float32), m, rtol=1e-5, atol=1e-6 * float(np.abs(m).max()), err_msg=f"step {step}: {part} m")
            np.testing.assert_allclose(ext.read_device(getattr(B, f"{part}_v"), w.shape, np.float32), v, rtol=1e-5, atol=1e-6 * float(np.abs(v).max()), err_msg=f"step {step}: {part} v")


def _assert_update_skipped(t, before, what):
    st = t.stats()
    assert st.skipped == 1, f"{what}: update not skipped"
    after = _optimizer_state(t)
    for k in ("table_f32", "table_m", "table_v", "mlp_f32", "mlp_m", "mlp_v"):
        assert np.array_equal(after[k].view(np.uint32), before[k].view(np.uint32)), f"{what}: {k} changed"
    m, _ = t.model()
    E = before["table_f32"].size
    assert np.array_equal(ext.read_device(m.table, (E,), np.float16), before["table_f32"].astype(np.float16)), f"{what}: fp16 table changed"
    return st


def test_adam_guard_skips_update(dataset):
    """A gradient norm above the guard skips the update (:1515) and leaves
    weights and moments as they were; the step still counts."""
    announce("train adam: guard skip")
    hyper = ext.hyper_params(clip=1e30, guard=1e-9, loss_scale=LOSS_SCALE)
    t, _ = _trainer(dataset, hyper=hyper)
    t.step(1)  # first step: skipped as well (moments stay zero)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
    t.synchronize()
    before = _optimizer_state(t)
    assert _grad_norm(before) > 1e-9
    t.run_stages(L.NERF_EXT_STAGE_ADAM, L.NERF_EXT_STAGE_END)
    st = _assert_update_skipped(t, before, "guard")
    assert st.last.has_nonfinite == 0
    assert st.last.completed_steps == 2


def test_nonfinite_gradient_skips_update(dataset):
    """A NaN in one sample's loss gradient reaches the weight and table
    gradients: the step reports has_nonfinite = 1 and skips the update
    (:1462-1476, :1501, :1518)."""
    announce("train adam: NaN gradient skip")
    t, _ = _trainer(dataset)
    t.step(1)
    t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_COMPOSITE)
    t.synchronize()
    before = _optimizer_state(t)
    B = t.buffers()
    ext.write_device(B.draw, np.array([np.nan, 0.0, 0.0, 0.0], np.float32))
    t.run_stages(L.NERF_EXT_STAGE_BACKWARD, L.NERF_EXT_STAGE_END)
    st = _assert_update_skipped(t, before, "NaN")
    assert st.last.has_nonfinite == 1
    assert st.last.completed_steps == 2
    # The next step trains normally again.
    t.step(1)
    st = t.stats()
    assert st.skipped == 0 and st.last.has_nonfinite == 0


# 20,000 cells: whole bit words (one launch evaluates, decays and sets the
# bits); 20,001: the window's edges split words (a bit pass of its own).
@pytest.mark.parametrize("count", [20000, 20001])
def test_occupancy_window_rotates(dataset, count):
    """cells_per_update below the cell count: each refresh decays every cell
    and re-evaluates the window starting at frame x count mod cells, wrapping
    past the last cell (:1575-1627); two refreshes (frames 4 and 8)."""
    announce(f"train occupancy refresh, rotating window of {count}")
    cells = OCC_RES ** 3
    occ = ext.occupancy_params(warmup_steps=2, update_interval=4, cells_per_update=count, threshold=0.01, decay=0.95)
    t, grid = _trainer(dataset, occ=occ)
    B = t.buffers()
    idx = np.arange(cells)
    x, y, z = idx % OCC_RES, (idx // OCC_RES) % OCC_RES, idx // (OCC_RES * OCC_RES)
    step = np.float32(1.0 / OCC_RES)
    centres = np.stack([(x + 0.5) * step, (y + 0.5) * step, (z + 0.5) * step], 1).astype(np.float32)
    t.step(4)
    for frame in (4, 8):
        t.synchronize()
        table, dp, _ = _model_host(t)
        before = ext.read_device(B.density_grid, (cells,), np.float32)
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_OCCUPANCY)
        t.synchronize()
        got = ext.read_device(B.density_grid, (cells,), np.float32)
        start = frame * count % cells
        window = (start + np.arange(count)) % cells
        assert start + count > cells, "the window should wrap"
        want = before * np.float32(0.95)
        sigma = orc.density_forward(oracle_grid(grid), table, dp, centres[window])[:, 0]
        want[window] = np.maximum(want[window], sigma)
        outside = np.ones(cells, bool)
        outside[window] = False
        assert np.array_equal(got[outside], want[outside]), f"frame {frame}: cells outside the window are only decayed"
        assert_rel(got[window], want[window], what=f"frame {frame}: window cells")
        bits = ext.read_device(B.bitfield, (cells // 32,), np.uint32)
        want_bits = np.packbits((got > 0.01).reshape(-1, 32)[:, ::-1], axis=1).view(">u4").ravel().astype(np.uint32)
        assert np.array_equal(bits, want_bits), f"frame {frame}: bitfield != density > threshold"
        t.run_stages(L.NERF_EXT_STAGE_SAMPLE, L.NERF_EXT_STAGE_END)
        t.step(3)


def test_gradients_deterministic(dataset):
    """Two runs of the same step give bit-identical weight and table
    gradients: fixed-order partial sums and exact fixed-point bins, no
    order-dependent floating-point atomics on the gradient path."""
    announce("train gradients: run-to-run determinism")
    grads = []
    for _ in range(2):
        t, _ = _trainer(dataset, log2_table=17)
        t.step(2)
        t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_BACKWARD)
        t.synchronize()
        B = t.buffers()
        grads.append((ext.read_device(B.table_grad, (int(B.table_elems),), np.uint32), ext.read_device(B.mlp_grad, (10240,), np.uint32), ext.read_device(B.table_f32, (int(B.table_elems),), np.uint32)))
        t.close()
    assert np.array_equal(grads[0][2], grads[1][2]), "weights after two steps differ between runs"
    assert np.array_equal(grads[0][0], grads[1][0]), "table gradients differ between runs"
    assert np.array_equal(grads[0][1], grads[1][1]), "MLP weight gradients differ between runs"


def test_pipelined_steps_match_stage_by_stage(dataset):
    """Whole steps from one call (each step's begin and sampler overlapping
    the previous step's Adam on the trainer's second stream), whole steps
    one call each (the begin folded into the step's first kernel, the end
    into the backward's gradient-norm kernel) and every stage launched alone
    leave the same weights,
    moments, occupancy and step state bit for bit.  Ten steps cross the
    warm-up and two occupancy refreshes (frames 4 and 8), which wait for the
    previous Adam."""
    announce("train: pipelined steps vs whole steps vs single stages, 10 steps")
    runs = []
    for mode in ("pipelined", "steps", "stages"):
        t, _ = _trainer(dataset, log2_table=17, target_samples=RAYS * 24)
        if mode == "pipelined":
            t.step(10)
        elif mode == "steps":
            for _ in range(10):
                t.run_stages(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_END)
        else:
            for _ in range(10):
                for s in range(L.NERF_EXT_STAGE_BEGIN, L.NERF_EXT_STAGE_END + 1):
                    t.run_stages(s, s)
        st = t.stats()
        B = t.buffers()
        E = int(B.table_elems)
        cells = OCC_RES ** 3
        runs.append({"table_f32": ext.read_device(B.table_f32, (E,), np.uint32), "table_m": ext.read_device(B.table_m, (E,), np.uint32), "table_v": ext.read_device(B.table_v, (E,), np.uint32),
                     "mlp_f32": ext.read_device(B.mlp_f32, (10240,), np.uint32), "mlp_v": ext.read_device(B.mlp_v, (10240,), np.uint32),
                     "density": ext.read_device(B.density_grid, (cells,), np.uint32), "bits": ext.read_device(B.bitfield, (cells // 32,), np.uint32),
                     "completed_steps": st.last.completed_steps, "camera": st.last.last_train_camera, "rays": st.rays, "samples_total": st.samples_total, "skipped": st.skipped,
                     "has_nonfinite": st.last.has_nonfinite, "grad_norm": np.float32(st.last.grad_norm).view(np.uint32), "loss": st.last.loss})
        t.close()
    a = runs[0]
    assert a["completed_steps"] == 10
    for b, what in ((runs[1], "whole steps"), (runs[2], "single stages")):
        for k in a:
            if k == "loss":  # a sum of per-wave float atomics: its last bits follow the order they landed in
                assert abs(a[k] - b[k]) <= 1e-6 * abs(a[k]), f"loss differs between pipelined steps and {what}: {a[k]} vs {b[k]}"
            else:
                assert np.array_equal(np.asarray(a[k]), np.asarray(b[k])), f"{k} differs between pipelined steps and {what}: {a[k]} vs {b[k]}"
