"""nerf_bench, the host program on the reference ABI, end to end on the GPU:
training on the analytic scene and on a NeRF-synthetic directory written
here, its log lines, the periodic PSNR, the PNG it saves and a checkpoint
round trip through --save-weights / --load-weights (benchmark.cpp:305-546)."""
import json
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
EXE = ROOT / "nerf_amd" / "nerf_bench"
sys.path.insert(0, str(Path(__file__).resolve().parent))


def _run(args, timeout=180):
    if not EXE.exists():
        pytest.fail("nerf_bench is not built (run __graft_entry__.build())")
    p = subprocess.run([str(EXE), *args], capture_output=True, text=True, timeout=timeout)
    assert p.returncode == 0, f"nerf_bench failed ({p.returncode}): {p.stderr[-2000:]}"
    return p.stdout


def _evals(out):
    return [float(m) for m in re.findall(r"\[eval\] step=\d+ camera=\d+ psnr=([-+0-9.einf]+)", out)]


def test_synthetic_training_and_checkpoint(tmp_path):
    announce("nerf_bench --synthetic 8 (64x64), 60 steps")
    png, ckpt = tmp_path / "out.png", tmp_path / "w.safetensors"
    out = _run(["--synthetic", "8", "--synthetic-size", "64", "--steps", "60", "--rays", "1024", "--max-sample-steps", "64", "--log-interval", "20", "--inference-interval", "30",
                "--inference-out", str(png), "--save-weights", str(ckpt)])
    train = re.findall(r"\[train\] step=(\d+) loss=(\S+) loss_ema=\S+ grad_norm=(\S+) sps=(\S+) eta_sec=\S+ nonfinite=(\d)", out)
    assert [int(t[0]) for t in train] == [20, 40, 60]
    assert all(np.isfinite(float(t[1])) and t[4] == "0" for t in train)
    ev = _evals(out)
    assert len(ev) == 2 and all(np.isfinite(v) and v > 5.0 for v in ev)
    assert f"[eval] saved={png}" in out and png.stat().st_size > 64 * 64
    from test_harness import LIB_PATH  # noqa: F401  (libnerf_host.so decodes the PNG)
    import ctypes as C

    host = C.CDLL(str(LIB_PATH))
    data = png.read_bytes()
    w, h = C.c_uint32(), C.c_uint32()
    assert host.nerf_host_png_decode(data, C.c_uint64(len(data)), C.byref(w), C.byref(h), None, C.c_uint64(0)) == 0 and (w.value, h.value) == (64, 64)
    assert ckpt.exists()
    # Resume from the checkpoint: the first evaluation starts from trained weights.
    out2 = _run(["--synthetic", "8", "--synthetic-size", "64", "--steps", "1", "--rays", "1024", "--log-interval", "1", "--inference-interval", "1", "--inference-out", str(tmp_path / "b.png"),
                 "--load-weights", str(ckpt)])
    assert len(_evals(out2)) == 1


def test_dataset_directory(tmp_path):
    announce("nerf_bench --dataset (NeRF-synthetic layout written here), 20 steps")
    from test_harness import _png

    from helpers import ext

    # Frames rendered from the analytic scene, stored in the Blender frame:
    # invert the loader's transform (x, -z, y axes; x 0.33 + 0.5).
    g = ext.scene_gaussians(16, seed=2)
    cams = [ext.camera_orbit(3, i, 1.32, (0.5, 0.5, 0.5), 48, 48, 1111.0 * 48 / 800) for i in range(6)]
    imgs = ext.scene_render(g, cams, 128).numpy().view(np.uint8).reshape(6, 48, 48, 4)
    W = np.array([[1, 0, 0], [0, 0, 1], [0, -1, 0]], np.float64)
    (tmp_path / "train").mkdir()
    meta = {"camera_angle_x": float(2 * np.arctan(0.5 * 48 / cams[0].fx)), "frames": []}
    for i, c in enumerate(cams):
        m = np.array(c.c2w[:], np.float64).reshape(3, 4)
        blender = np.eye(4)
        blender[:3, :3] = W.T @ m[:, :3]
        blender[:3, 3] = W.T @ ((m[:, 3] - 0.5) / 0.33)
        (tmp_path / "train" / f"r_{i}.png").write_bytes(_png(imgs[i], 6, 6))
        meta["frames"].append({"file_path": f"./train/r_{i}", "transform_matrix": blender.tolist()})
    (tmp_path / "transforms_train.json").write_text(json.dumps(meta))
    out = _run(["--dataset", str(tmp_path), "--steps", "20", "--rays", "512", "--log-interval", "10", "--inference-interval", "20", "--inference-out", str(tmp_path / "o.png")])
    assert len(re.findall(r"\[train\] step=", out)) == 2
    ev = _evals(out)
    assert len(ev) == 1 and np.isfinite(ev[0])
