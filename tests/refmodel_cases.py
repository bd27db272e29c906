"""Inputs shared by the reference-model tests (oracle pins and GPU parity):
weight sets of the reference's own network (backend-cuda.cu:23-54) and
structured weights whose outputs have closed forms."""
import numpy as np

DENSITY_SHAPES = [(128, 64), (128, 128), (128, 128), (128, 128), (128, 128), (16, 128)]
COLOR_SHAPES = [(128, 48), (128, 128), (128, 128), (16, 128)]

# Position-encoding index of cos(4 y): level 2, slot 3 + 1 (:252-277 order
# x, y, z, then per level sin x, sin y, sin z, cos x, cos y, cos z).
POS_COS_4Y = 3 + 6 * 2 + 4
# Direction-encoding index of cos(dx) at level 0.
DIR_COS_X = 3 + 3


def pack(mats):
    return np.concatenate([m.ravel() for m in mats]).astype(np.float16).view(np.uint16)


def structured():
    """Density: hidden neuron 0 = relu(x), neuron 2 = relu(cos 4y), carried
    through identity hidden layers; raw output 0 <- neuron 2, raw output 1 <-
    neuron 0.  Colour: neuron 0 = relu(colour input 0) (geo feature 0 = raw
    density output 1), neuron 1 = relu(input 15 + DIR_COS_X), neuron 2 =
    input 47 (a padding column, always zero); raw colour c <- neuron c.
    Closed form for x > 0, |dx| < pi/2:
        raw = (cos 4y, x, cos dx, 0) as fp16 (each stage rounds to fp16)."""
    d = [np.zeros(s, np.float32) for s in DENSITY_SHAPES]
    d[0][0, 0] = 1.0
    d[0][2, POS_COS_4Y] = 1.0
    for m in d[1:5]:
        m[:, :] = np.eye(128)
    d[5][0, 2] = 1.0
    d[5][1, 0] = 1.0
    c = [np.zeros(s, np.float32) for s in COLOR_SHAPES]
    c[0][0, 0] = 1.0
    c[0][1, 15 + DIR_COS_X] = 1.0
    c[0][2, 47] = 1.0
    for m in c[1:3]:
        m[:, :] = np.eye(128)
    for k in range(3):
        c[3][k, k] = 1.0
    return pack(d), pack(c)


def structured_raw(pos, dirs):
    f16 = lambda v: np.asarray(v, np.float32).astype(np.float16).astype(np.float32)
    cos4y = f16(np.cos(np.float64(pos[:, 1].astype(np.float32) * np.float32(4.0))))
    return np.stack([np.maximum(cos4y, 0), f16(pos[:, 0]), f16(np.cos(np.float64(dirs[:, 0]))), np.zeros(len(pos), np.float32)], 1)


def world_points(n, seed, lo=-1.5, hi=1.5):
    return np.random.default_rng(seed).uniform(lo, hi, (n, 3)).astype(np.float32)


def unit_dirs(n, seed):
    v = np.random.default_rng(seed).normal(size=(n, 3))
    return (v / np.linalg.norm(v, axis=1, keepdims=True)).astype(np.float32)
