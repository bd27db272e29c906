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


def pos_entry(level, kind, axis):
    """Position-encoding index of sin (kind 0) / cos (kind 1) of 2^level
    times coordinate `axis`."""
    return 3 + 6 * level + 3 * kind + axis


def encoding_probe(d_entry, c_entries, c_from_dir):
    """Weights whose four raw outputs are four frequency-encoding values:
    raw density 0 = position entry d_entry, raw colour k = position entry
    c_entries[k] (carried through raw density output k + 1, the colour
    input's geometry column k) or, with c_from_dir, direction entry
    c_entries[k].  Each value v enters as the neuron pair relu(v), relu(-v),
    identity hidden layers carry both, and the linear output layer takes
    their difference: every product is 1 x an fp16 value and every sum has
    one nonzero term, so the raw outputs are the encoding's fp16 values
    exactly."""
    d = [np.zeros(s, np.float32) for s in DENSITY_SHAPES]
    c = [np.zeros(s, np.float32) for s in COLOR_SHAPES]
    d[0][0, d_entry], d[0][1, d_entry] = 1.0, -1.0
    d[5][0, 0], d[5][0, 1] = 1.0, -1.0
    for k in range(3):
        if not c_from_dir:
            d[0][2 + 2 * k, c_entries[k]], d[0][3 + 2 * k, c_entries[k]] = 1.0, -1.0
            d[5][1 + k, 2 + 2 * k], d[5][1 + k, 3 + 2 * k] = 1.0, -1.0
        col = 15 + c_entries[k] if c_from_dir else k
        c[0][2 * k, col], c[0][2 * k + 1, col] = 1.0, -1.0
        c[3][k, 2 * k], c[3][k, 2 * k + 1] = 1.0, -1.0
    for m in d[1:5] + c[1:3]:
        m[:, :] = np.eye(128)
    return pack(d), pack(c)


def encoding_values(v, levels):
    """Frequency encoding of rows v [n][3] in numpy: sin and cos evaluated in
    fp64 on the exact fp32 argument v 2^l, rounded to fp32, then to fp16."""
    v = np.asarray(v, np.float32)
    cols = [v[:, a].astype(np.float64) for a in range(3)]
    for l in range(levels):
        arg = [(v[:, a] * np.float32(2.0 ** l)).astype(np.float64) for a in range(3)]
        cols += [np.sin(x) for x in arg] + [np.cos(x) for x in arg]
    e = np.stack(cols, 1).astype(np.float32).astype(np.float16).astype(np.float32)
    return e


def encoding_probe_raw(pos, dirs, d_entry, c_entries, c_from_dir):
    pe, de = encoding_values(pos, 10), encoding_values(dirs, 4)
    src = de if c_from_dir else pe
    return np.stack([pe[:, d_entry]] + [src[:, k] for k in c_entries], 1)


# (density entry, three colour entries, colour entries from the direction):
# sine and cosine on the finest levels (|2^9 x| up to 768) and the coarsest,
# both networks, every axis.
ENCODING_PROBES = [
    (pos_entry(9, 0, 0), [pos_entry(9, 1, 1), pos_entry(8, 0, 2), pos_entry(7, 1, 0)], False),
    (pos_entry(9, 1, 2), [pos_entry(0, 0, 1), pos_entry(3, 1, 0), pos_entry(5, 0, 2)], False),
    (pos_entry(6, 0, 1), [3 + 6 * 3 + 2, 3 + 6 * 3 + 3, 3 + 6 * 2 + 4], True),
    (1, [0, 3 + 1, 3 + 6 * 1 + 5], True),
]


def probe_points(n, seed):
    """World points over the scene box plus edge values (0, the box faces,
    tiny magnitudes, both signs)."""
    p = world_points(n, seed)
    edge = np.array([[0.0, -0.0, 1.5], [-1.5, 1e-7, -1e-7], [1.0, -1.0, 0.5], [np.pi / 4, np.pi / 2, -np.pi]], np.float32)
    return np.concatenate([p, edge])


def world_points(n, seed, lo=-1.5, hi=1.5):
    return np.random.default_rng(seed).uniform(lo, hi, (n, 3)).astype(np.float32)


def unit_dirs(n, seed):
    v = np.random.default_rng(seed).normal(size=(n, 3))
    return (v / np.linalg.norm(v, axis=1, keepdims=True)).astype(np.float32)
