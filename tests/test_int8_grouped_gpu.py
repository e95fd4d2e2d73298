"""Parity of the int8 products with a scale per row and 128 columns: the reference's default load mode (a bf16
checkpoint requantized at load, src/cuda/core.rs:338-389, multiplied by kernels/gemm.cuh:176-200) and pre-quantized
group-128 int8 checkpoints. Unlike per-channel int8 (one scale per row: exact integer prefill products), these run the
prefill kernel's per-group dequantization (each weight (q - 128) s rounded once to bf16), so every test first checks
that the matrix is not taken for per-channel.

Matrices are built both ways the loader builds them: Mat.new(int8=True) over dense bf16 weights (the requantization,
max|w| / 127 per row and 128 columns) and Mat.stack over a stored int8 Quant with group 128. Outputs are checked on a
sample of rows at the 27B shapes: decode sizes (the skinny kernel) are exact products, 1e-4 of RMS against the f64
oracle; prefill sizes 1e-4 against the f64 product of bf16-rounded weights and 2e-2 (the north star's bar) against
the oracle. Argmax runs at the same bars; SwiGLU as its test says.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import SKINNY_MAX_M, Epi, Mat, Wt
from qwenny_amd.core import Quant
from qwenny_amd.synth import activations, f32_to_bf16
from tests.helpers import (TOL, bf16_out_err, emulate_bf16_weights, emulate_silu_prefill, make_quant, oracle_y, rel_err,
                           silu_bar, sub_quant, to_dev)

pytestmark = pytest.mark.gpu

SHAPES = [(5120, 17408), (17408, 5120)]  # (K, N)
MS = [1, 5, 17, 48, 49, 130, 256, 2048]


def dense_weights(seed, n, k):
    """bf16 weights [n][k] ~ N(0, 0.05^2), with every 7th row 10x larger, so per-group scales vary widely."""
    w = np.random.default_rng(seed).standard_normal((n, k), dtype=np.float32) * 0.05
    w[::7] *= 10.0
    return f32_to_bf16(w)


def requant_quant(w_bf16):
    """The int8 Quant the load-time requantization makes of dense bf16 weights (oracle.requant_int8: stored q + 128,
    scale per row and 128 columns; w = (q - 128) s)."""
    n, k = w_bf16.shape
    vals, sc = oracle.requant_int8(w_bf16)
    sc = sc.reshape(-1)
    return Quant(8, 128, n, k, vals.view(np.uint32).reshape(n, k // 4), sc, -128.0 * sc)


_cache = {}


def _mats(gemm, way, k, n):
    """(Mat, the Quant it holds) for one of the two construction ways, built once per shape."""
    key = (way, k, n)
    if key not in _cache:
        _cache.clear()  # one shape's matrices at a time (host memory)
        if way == "checkpoint":
            q = make_quant(700 + k % 97, "i8g", n, k)
            mat = Mat.stack(gemm, [q])
        else:
            w = dense_weights(710 + k % 97, n, k)
            q = requant_quant(w)
            mat = Mat.new(gemm, w, k, int8=True)
        _cache[key] = (mat, q)
    return _cache[key]


def _plain(gemm, mat, x, m):
    import torch

    split = mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
    torch.cuda.synchronize()
    parts = y.cpu().numpy().astype(np.float64)
    assert not np.isnan(parts).any()
    return parts.sum(0)


@pytest.mark.parametrize("way", ["checkpoint", "requant"])
@pytest.mark.parametrize("k,n", SHAPES)
@pytest.mark.parametrize("m", MS)
def test_grouped_int8_plain(gemm, way, k, n, m):
    print(f"grouped int8 plain {way} K={k} N={n} m={m}", flush=True)
    mat, q = _mats(gemm, way, k, n)
    assert mat.wt == Wt.I8 and not mat.per_channel
    x = activations(720 + m, "x", m, k, outliers=0.01 if m > SKINNY_MAX_M else 0.0)
    rows = np.sort(np.random.default_rng(m).choice(n, 64 if m >= 256 else 256, replace=False))
    sq = sub_quant(q, rows)
    got = _plain(gemm, mat, x, m)[:, rows]
    want = oracle_y(sq, x)
    if mat.kernel(m) == "skinny":
        assert rel_err(got, want) <= 1e-4
    else:
        assert rel_err(got, want) <= TOL
        assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4


@pytest.mark.parametrize("way", ["checkpoint", "requant"])
@pytest.mark.parametrize("m", [5, 48, 256])
def test_grouped_int8_silu(gemm, way, m):
    """SwiGLU over the 27B [gate; up] (2 x 17408 rows, K 5120), checked on a sample of 256 outputs: decode sizes
    against the oracle, prefill sizes against the kernel's arithmetic (bf16-rounded weights)."""
    import torch

    print(f"grouped int8 silu {way} m={m}", flush=True)
    _cache.clear()
    n, k = 17408, 5120
    if way == "checkpoint":
        gate, up = make_quant(730, "i8g", n, k), make_quant(731, "i8g", n, k)
        mat = Mat.stack(gemm, [gate, up], silu=True)
    else:
        wg, wu = dense_weights(732, n, k), dense_weights(733, n, k)
        gate, up = requant_quant(wg), requant_quant(wu)
        mat = Mat.new(gemm, np.concatenate([wg, wu]), k, silu=True, int8=True)
    assert mat.wt == Wt.I8 and not mat.per_channel
    x = activations(734 + m, "x", m, k)
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    cols = np.sort(np.random.default_rng(m).choice(n, 256, replace=False))
    got = y.float().cpu().numpy()[:, cols]
    sg, su = sub_quant(gate, cols), sub_quant(up, cols)
    if mat.kernel(m, Epi.Silu) == "skinny":
        g, u = oracle_y(sg, x), oracle_y(su, x)
        tol = TOL
    else:
        g, u = emulate_silu_prefill(sg, x), emulate_silu_prefill(su, x)
        # the epilogue's inputs carry each weight's f16 rounding and the activations' conversion to f16; the epilogue
        # is checked against silu over that arithmetic
        tol = 1e-3
    assert bf16_out_err(got, g / (1.0 + np.exp(-g)) * u) <= tol
    # both kernels against the oracle's exact product: the product bar carried through the epilogue, and the bar of
    # the output itself
    eg, eu = oracle_y(sg, x), oracle_y(su, x)
    assert silu_bar(got, eg, eu) <= 1.0
    assert bf16_out_err(got, eg / (1.0 + np.exp(-eg)) * eu) <= TOL


@pytest.mark.parametrize("way", ["checkpoint", "requant"])
@pytest.mark.parametrize("n_out", [1, 5, 64])
def test_grouped_int8_argmax(gemm, way, n_out):
    """The argmax epilogue over a (5120, 17408) grouped int8 matrix, logit rows gathered from 100 token rows: keys
    exactly those of the written logits, logits at the bar of their kernel."""
    import torch

    print(f"grouped int8 argmax {way} n_out={n_out}", flush=True)
    k, n, steps = 5120, 17408, 100
    mat, q = _mats(gemm, way, k, n)
    x = activations(740 + n_out, "x", steps, k)
    rows = np.random.default_rng(n_out).choice(steps, n_out, replace=False).astype(np.int32)
    y = torch.zeros((n_out, n), dtype=torch.float32, device="cuda")
    keys = torch.zeros(n_out, dtype=torch.int64, device="cuda")
    gemm.run(None, steps, mat, to_dev(x), y, Epi.Argmax, out_rows=torch.from_numpy(rows).cuda(), n_out=n_out,
             keys=keys)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert (keys.cpu().numpy().view(np.uint64) == oracle.argmax_keys(got, n)).all()
    samp = np.sort(np.random.default_rng(1).choice(n, 512, replace=False))
    sq = sub_quant(q, samp)
    want = oracle_y(sq, x[rows])
    if mat.kernel(n_out, Epi.Argmax) == "skinny":
        assert rel_err(got[:, samp], want) <= 1e-4
    else:
        assert rel_err(got[:, samp], want) <= TOL
        assert rel_err(got[:, samp], emulate_bf16_weights(sq, x[rows])) <= 1e-4
