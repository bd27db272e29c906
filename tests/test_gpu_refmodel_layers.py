"""Reference-model network pinned layer by layer on the GPU's own rows.

Ten fp16-rounded 128-wide layers carry a rounding-tie flip (the GPU's fp32
accumulation and the oracle's fp64 sum on either side of an fp16 tie) into
every later layer, which is why the end-to-end comparisons of raw outputs
are statistical.  Here each layer is checked on its own: the backward
(nerf_ext_ref_backward_rows) leaves the fp16 input of every layer and the
fp16 delta of every layer's output; each layer's output is recomputed in
fp64 from the GPU's stored input of that layer with the fp16 weights
(backend-cuda.cu:668-835 forward, :784-909 backward semantics: no bias,
ReLU, [out][in] weights, fp16 rounding of every activation and delta), and
must equal the GPU's stored next row within one fp16 ulp (or, where
cancellation makes the fp32 sum's own error larger, within Higham's bound
gamma_k sum |w x| on it), with at least 99.9 % bit-identical.  The forward kernel's raw outputs
(nerf_ext_ref_field_forward) are checked the same way against the output
layers applied to the backward's rows, the encodings against the oracle's
frequency encoding, and the weight gradients against fp64 sums of the
GPU's own delta x input rows.
"""
import numpy as np
import pytest

from conftest import announce
from helpers import L, ext, orc, DeviceArray, synchronize
from refmodel_cases import COLOR_SHAPES, DENSITY_SHAPES, unit_dirs, world_points

pytestmark = pytest.mark.gpu

ACT_OFF = [0, 64, 192, 320, 448, 576, 704, 752, 880, 1008]
DLT_OFF = [0, 128, 256, 384, 512, 640, 656, 784, 912, 1040]
ACT_ROWS, DLT_ROWS = 1136, 1056
SHAPES = DENSITY_SHAPES + COLOR_SHAPES  # layers 0..5 density, 6..9 colour
LOSS_SCALE = 128.0


def _rows(buf: np.ndarray, rows: int, n: int) -> np.ndarray:
    """[rows][n] float64 from the neuron-major layout (blocks of 32 samples)."""
    np_ = buf.size // rows
    return buf.view(np.float16).reshape(np_ // 32, rows, 32).transpose(1, 0, 2).reshape(rows, np_)[:, :n].astype(np.float64)


def _weights(model):
    d = model.density.numpy().astype(np.float64)
    c = model.color.numpy().astype(np.float64)
    out, off = [], 0
    for o, i in DENSITY_SHAPES:
        out.append(d[off:off + o * i].reshape(o, i))
        off += o * i
    off = 0
    for o, i in COLOR_SHAPES:
        out.append(c[off:off + o * i].reshape(o, i))
        off += o * i
    return out


def _ulps(got: np.ndarray, want_f64: np.ndarray) -> np.ndarray:
    """Distance in fp16 ulps between fp16 values and fp16(want), as ordered
    integers (so -0 and +0 are one apart only if they differ in sign)."""
    def key(x):
        b = x.astype(np.float16).view(np.int16).astype(np.int64)
        return np.where(b < 0, -(b & 0x7FFF), b)
    return np.abs(key(got) - key(want_f64))


def _check(got, want, what, sabs=None, k=0):
    """got (fp16 values) against fp16(want): at most one ulp apart, or, for a
    value the GPU summed over k products in fp32, within half an fp16 ulp
    plus Higham's bound on fp32 summation, gamma_k sum |w x| (sabs), which
    cancellation can push past one fp16 ulp of a small result; at least
    99.9 % bit-identical."""
    u = _ulps(got, want)
    ok = u <= 1
    if sabs is not None:
        gamma = k * 2.0 ** -24 / (1.0 - k * 2.0 ** -24)
        g16 = got.astype(np.float16)
        half_ulp = 0.5 * np.abs(np.spacing(g16).astype(np.float64))
        ok |= np.abs(got - want) <= half_ulp + gamma * sabs
    exact = float(np.mean(u == 0))
    print(f"[layer] {what}: {exact * 100:.3f} % bit-identical, max {int(u.max())} ulp ({int(np.count_nonzero(u > 1))} beyond one, within the fp32 summation bound)", flush=True)
    assert ok.all(), f"{what}: {int(np.count_nonzero(~ok))} values beyond one fp16 ulp and the fp32 summation bound (max {int(u.max())} ulp)"
    assert exact >= 0.999, f"{what}: only {exact:.4%} bit-identical"


@pytest.mark.parametrize("scale,n", [(1.5, 5000), (1.0, 9000)])
def test_ref_layers_from_gpu_rows(scale, n):
    announce(f"reference-model network layer by layer, weights x {scale}, n={n}")
    m = ext.RefModel.create(ext.ref_mlp_init(0) * scale, ext.ref_mlp_init(1) * scale)
    pos, dirs = world_points(n, 51), unit_dirs(n, 52)
    draw = np.random.default_rng(53).normal(0, 1e-2, (n, 4)).astype(np.float32)
    np_ = (n + 63) // 64 * 64
    d_p, d_d, d_r = DeviceArray.from_numpy(pos), DeviceArray.from_numpy(dirs), DeviceArray.from_numpy(draw)
    acts, dlts = DeviceArray((ACT_ROWS * np_,), np.uint16), DeviceArray((DLT_ROWS * np_,), np.uint16)
    gD, gC = DeviceArray((75776,), np.float32), DeviceArray((40960,), np.float32)
    out, raw = DeviceArray((n, 4), np.float32), DeviceArray((n, 4), np.float32)
    L.call("nerf_ext_ref_backward_rows", m.density.ptr, m.color.ptr, d_p.ptr, d_d.ptr, d_r.ptr, n, LOSS_SCALE, gD.ptr, gC.ptr, acts.ptr, dlts.ptr, None)
    L.call("nerf_ext_ref_field_forward", m.density.ptr, m.color.ptr, d_p.ptr, d_d.ptr, n, out.ptr, raw.ptr, None)
    synchronize()
    A = _rows(acts.numpy(), ACT_ROWS, n)
    D = _rows(dlts.numpy(), DLT_ROWS, n)
    W = _weights(m)
    raw = raw.numpy().astype(np.float64)
    inp = lambda l: A[ACT_OFF[l]:ACT_OFF[l] + SHAPES[l][1]]

    # Encodings: the oracle's frequency encoding (fp64 sin/cos), fp16.
    pe = orc.freq_encode(pos, 10).T.astype(np.float64)
    de = orc.freq_encode(dirs, 4).T.astype(np.float64)
    _check(inp(0)[:63], pe, "position encoding (layer 0 input)")
    assert np.all(inp(0)[63] == 0)
    _check(inp(6)[15:42], de, "direction encoding (layer 6 input)")
    assert np.all(inp(6)[42:] == 0)

    # Forward, one layer at a time from the GPU's own input rows.
    fwd_abs = lambda l: np.abs(W[l]) @ np.abs(inp(l))
    for l in (0, 1, 2, 3, 4, 6, 7, 8):
        _check(inp(l + 1), np.maximum(W[l] @ inp(l), 0.0), f"layer {l} -> {l + 1} activations", fwd_abs(l), SHAPES[l][1])
    z5, a5 = W[5] @ inp(5), fwd_abs(5)
    _check(inp(6)[:15], z5[1:16], "density outputs 1..15 (colour input)", a5[1:16], 128)
    _check(raw[:, 0], z5[0], "raw density (forward kernel)", a5[0], 128)
    z9, a9 = W[9] @ inp(9), fwd_abs(9)
    _check(raw[:, 1:].T, z9[:3], "raw colour (forward kernel)", a9[:3], 128)

    # Backward: deltas layer by layer from the GPU's own deltas and ReLU masks.
    dl = lambda l: D[DLT_OFF[l]:DLT_OFF[l] + SHAPES[l][0]]
    ls = np.float32(LOSS_SCALE)
    want9 = np.zeros((16, n))
    want9[:3] = (ls * draw[:, 1:]).T
    _check(dl(9), want9, "colour output deltas (fp16 of loss_scale d raw)")
    bwd_abs = lambda l: np.abs(W[l + 1].T) @ np.abs(dl(l + 1))
    for l in (8, 7, 6, 4, 3, 2, 1, 0):
        if l == 4:
            want5 = np.zeros((16, n))
            want5[0] = ls * draw[:, 0]
            want5[1:] = (W[6].T @ dl(6))[:15]
            a5 = np.zeros((16, n))
            a5[1:] = (np.abs(W[6].T) @ np.abs(dl(6)))[:15]
            _check(dl(5), want5, "density output deltas (loss_scale d raw sigma, geometry deltas)", a5, 128)
        _check(dl(l), (inp(l + 1) > 0) * (W[l + 1].T @ dl(l + 1)), f"layer {l} deltas from layer {l + 1}", bwd_abs(l), SHAPES[l + 1][0])

    # Weight gradients: fp64 sums of the GPU's delta x input rows.
    g = np.concatenate([gD.numpy(), gC.numpy()]).astype(np.float64)
    off = 0
    for l, (o, i) in enumerate(SHAPES):
        want = dl(l) @ inp(l).T
        got = g[off:off + o * i].reshape(o, i)
        off += o * i
        rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
        print(f"[layer] dW layer {l}: relative Frobenius {rel:.3e}", flush=True)
        assert rel <= 1e-4, f"dW layer {l}: relative Frobenius error {rel:.3e}"
