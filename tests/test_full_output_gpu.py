"""Whole outputs of BASELINE.json's prefill configurations (configs[3] int4 with and without zero points, configs[4]
per-channel int8) at their full sizes: every output of every item, stream-K cut items and K slices included, against
an independent CPU product of the same stored matrix. The weights are dequantized in numpy from the stored codes,
scales and offsets (w = q s + offset, the Quant semantics of src/checkpoint.rs:39-47, in f64) and multiplied by BLAS:
- against the exact f64 product, the north star's bar, max |err| <= 2e-2 RMS(output);
- against the same product over each weight rounded once to bf16 (the prefill kernel's arithmetic by design), 1e-4;
  per-channel int8 keeps exact integer weights (scale after the sum) and is held to 1e-4 of the exact product.
The decode layer set is covered the same way at M = 1 and 5."""

import numpy as np
import pytest

from qwenny_amd import Epi, Mat, Wt
from qwenny_amd.synth import activations, bf16_to_f32
from tests.helpers import TOL, make_quant, to_dev

pytestmark = pytest.mark.gpu

PREFILL_27B = [(5120, 17408), (17408, 5120), (5120, 6144)]
SET_27B = [(5120, 17408), (17408, 5120), (5120, 6144), (6144, 5120)]


class _Dequant:
    """Rows of a stored matrix dequantized in f64, q s + offset per (row, group) from the packed words, a block of
    rows at a time into reused buffers (large fresh allocations are slow on some hosts)."""

    def __init__(self, q, block):
        self.q, self.block = q, block
        self.per, self.g = 32 // q.bits, q.cols // q.group
        self.shifts = np.arange(self.per, dtype=np.uint32) * q.bits
        self.mask = np.uint32((1 << q.bits) - 1)
        self.codes = np.empty((block, q.q.shape[1], self.per), np.uint32)
        self.w = np.empty((block, self.g, q.group), np.float64)
        self.f32 = np.empty((block, q.cols), np.float32)

    def rows(self, r0, r1):
        q, n = self.q, r1 - r0
        codes = self.codes[:n]
        np.right_shift(q.q[r0:r1, :, None], self.shifts, out=codes)
        np.bitwise_and(codes, self.mask, out=codes)
        w = self.w[:n]
        w[...] = codes.reshape(n, self.g, q.group)
        w *= q.scales.reshape(q.rows, self.g, 1)[r0:r1]
        w += q.offsets.reshape(q.rows, self.g, 1)[r0:r1]
        return w.reshape(n, q.cols)

    def bf16(self, w):
        """w rounded to f32, then to bf16 (nearest even), in place: each weight as the prefill kernel uses it ((q - z) s
        rounded once in f32, then to bf16; finite values only)."""
        f = self.f32[:len(w)]
        f[...] = w
        u = f.view(np.uint32)
        u += np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))
        u &= np.uint32(0xFFFF0000)
        w[...] = f
        return w


def _whole_check(got, q, x, exact_bar, emul_bar):
    """max |got - want| / RMS(want) over every output, want the exact f64 product (and, if emul_bar, the product over
    bf16-rounded weights), computed 256 rows at a time."""
    xf = bf16_to_f32(x).astype(np.float64)
    m, block = x.shape[0], 256
    dq = _Dequant(q, block)
    yb = np.empty((m, block), np.float64)
    worst = [0.0, 0.0]
    ss = [0.0, 0.0]
    for r0 in range(0, q.rows, block):
        r1 = min(q.rows, r0 + block)
        w = dq.rows(r0, r1)
        for i, bar in enumerate((exact_bar, emul_bar)):
            if bar is None:
                continue
            if i == 1:
                w = dq.bf16(w)
            y = yb[:, :r1 - r0]
            np.matmul(xf, w.T, out=y)
            worst[i] = max(worst[i], float(np.abs(got[:, r0:r1] - y).max()))
            ss[i] += float(np.einsum("ij,ij->", y, y))
    for i, bar in enumerate((exact_bar, emul_bar)):
        if bar is not None:
            rms = np.sqrt(ss[i] / (m * q.rows))
            assert worst[i] / rms <= bar, (i, worst[i] / rms)


def _product(gemm, mat, x, m):
    import torch

    split = mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
    torch.cuda.synchronize()
    got = (y[0] if split == 1 else y.double().sum(0)).cpu().numpy()
    assert not np.isnan(got).any()
    return got


def _check_prefill(gemm, q, x, m, exact_int):
    mat = Mat.stack(gemm, [q])
    got = _product(gemm, mat, x, m)
    if exact_int:
        _whole_check(got, q, x, 1e-4, None)
    else:
        _whole_check(got, q, x, TOL, 1e-4)
    return mat


@pytest.mark.parametrize("shape", PREFILL_27B)
@pytest.mark.parametrize("kind", ["i4", "i4z"])
def test_config3_whole_output_m2048(gemm, kind, shape):
    k, n = shape
    print(f"configs[3] whole output {kind} {n}x{k} m=2048", flush=True)
    q = make_quant(450 + k % 97, kind, n, k)
    x = activations(460 + k % 89, "x", 2048, k, outliers=0.01)
    mat = _check_prefill(gemm, q, x, 2048, False)
    assert mat.wt == (Wt.I4Z if kind == "i4z" else Wt.I4)


@pytest.mark.parametrize("m", [256, 512])
def test_config3_whole_output_short(gemm, m):
    """256 and 512 tokens: K-sliced partials and stream-K, every output."""
    for k, n in PREFILL_27B:
        print(f"configs[3] whole output i4z {n}x{k} m={m}", flush=True)
        q = make_quant(470 + k % 97, "i4z", n, k)
        x = activations(480 + m, "x", m, k, outliers=0.01)
        _check_prefill(gemm, q, x, m, False)


@pytest.mark.parametrize("shape", [(5120, 17408), (17408, 5120)])
def test_config4_whole_output_m2048(gemm, shape):
    k, n = shape
    print(f"configs[4] whole output int8 per channel {n}x{k} m=2048", flush=True)
    q = make_quant(490 + k % 97, "i8", n, k)
    x = activations(495 + k % 89, "x", 2048, k)
    mat = _check_prefill(gemm, q, x, 2048, True)
    assert mat.wt == Wt.I8 and mat.per_channel


@pytest.mark.parametrize("m", [1, 5])
def test_config2_whole_output(gemm, m):
    """The decode layer set: exact products, every output within 1e-4 of RMS of the f64 product."""
    for k, n in SET_27B:
        print(f"configs[2] whole output {n}x{k} m={m}", flush=True)
        q = make_quant(440 + k % 97, "i4", n, k)
        x = activations(445 + m, "x", m, k)
        _whole_check(_product(gemm, Mat.stack(gemm, [q]), x, m), q, x, 1e-4, None)
