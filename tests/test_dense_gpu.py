"""Parity of the dense 16-bit products (the reference's Wt::F16: Mat::new with int8 off, and the 16-bit matrices a
pre-quantized checkpoint keeps, such as the DeltaNet in_ba projection) through the C ABI.

The weights stay bf16 (QH_WT_BF16). Both kernels multiply them exactly in f32 (bf16 x bf16 products are exact), so the
outputs match the f64 oracle of the bf16 weights to 1e-4 of RMS; against the reference's own semantics, which rounds
the weights to f16 (exact for bf16 values in f16's normal range), the bar is the north star's 2e-2 RMS.
"""

import json

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, Wt, row_order
from qwenny_amd.checkpoint import Checkpoint, save_safetensors
from qwenny_amd.synth import activations, bf16_to_f32, f32_to_bf16
from tests.helpers import TOL, bf16_out_err, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _weights(seed, rows, cols):
    w = np.random.default_rng(seed).standard_normal((rows, cols)).astype(np.float32) * 0.05
    return f32_to_bf16(w)


def _plain(gemm, mat, x, m):
    import torch

    split = mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
    torch.cuda.synchronize()
    return y.sum(0).cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 130, 300])
def test_dense_plain(gemm, m):
    print(f"dense plain m={m}", flush=True)
    rows, cols = 384, 1024
    w = _weights(51 + m, rows, cols)
    x = activations(52 + m, "x", m, cols, outliers=0.01)
    mat = Mat.new(gemm, w, cols, int8=False)
    assert mat.wt == Wt.BF16 and mat.rows == rows
    got = _plain(gemm, mat, x, m)
    assert rel_err(got, oracle.dense_f64(w, x)) <= 1e-4
    assert rel_err(got, oracle.dense_f64(w, x, f16_weights=True)) <= TOL


@pytest.mark.parametrize("m", [64, 200])
def test_dense_k_sliced(gemm, m):
    """A short dense prefill product cut into K slices: several partials, each written, summing to the product."""
    print(f"dense K-sliced m={m}", flush=True)
    rows, cols = 1024, 4096
    w = _weights(56 + m, rows, cols)
    x = activations(57 + m, "x", m, cols, outliers=0.01)
    mat = Mat.new(gemm, w, cols, int8=False)
    assert mat.split(m) > 1
    got = _plain(gemm, mat, x, m)
    assert not np.isnan(got).any()
    assert rel_err(got, oracle.dense_f64(w, x)) <= 1e-4


@pytest.mark.parametrize("m", [1, 5, 300])
def test_dense_in_ba_shape(gemm, m):
    """The 27B DeltaNet in_ba projection (K 5120, N 96), which stays 16-bit in a pre-quantized checkpoint: 6 tiles,
    fewer than any wave column or prefill workgroup covers."""
    print(f"dense in_ba m={m}", flush=True)
    rows, cols = 96, 5120
    w = _weights(71 + m, rows, cols)
    x = activations(72 + m, "x", m, cols)
    mat = Mat.new(gemm, w, cols, int8=False)
    got = _plain(gemm, mat, x, m)
    assert rel_err(got, oracle.dense_f64(w, x)) <= 1e-4


@pytest.mark.parametrize("m", [1, 40])
def test_dense_silu(gemm, m):
    import torch

    print(f"dense silu m={m}", flush=True)
    n, k = 512, 768
    gate, up = _weights(61, n // 2, k), _weights(62, n // 2, k)
    x = activations(63, "x", m, k)
    mat = Mat.new(gemm, np.concatenate([gate, up]), k, silu=True, int8=False)
    y = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    full = np.concatenate([oracle.dense_f64(gate, x), oracle.dense_f64(up, x)], axis=1)
    want = oracle.silu_glu(full, row_order(n, True))
    assert bf16_out_err(y.float().cpu().numpy(), want) <= 1e-3


@pytest.mark.parametrize("n_out", [3, 40])
def test_dense_argmax(gemm, n_out):
    import torch

    print(f"dense argmax n_out={n_out}", flush=True)
    n, k, steps = 1024, 512, 50
    w = _weights(71, n, k)
    x = activations(72, "x", steps, k)
    rows = np.random.default_rng(4).choice(steps, n_out, replace=False).astype(np.int32)
    mat = Mat.new(gemm, w, k, int8=False)
    y = torch.zeros((n_out, n), dtype=torch.float32, device="cuda")
    keys = torch.zeros(n_out, dtype=torch.int64, device="cuda")
    gemm.run(None, steps, mat, to_dev(x), y, Epi.Argmax, out_rows=torch.from_numpy(rows).cuda(), n_out=n_out,
             keys=keys)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert rel_err(got, oracle.dense_f64(w, x[rows])) <= 1e-4
    assert (keys.cpu().numpy().view(np.uint64) == oracle.argmax_keys(got, n)).all()


@pytest.mark.parametrize("prequantized", [True, False])
def test_dense_from_checkpoint(gemm, tmp_path, prequantized):
    """Mat.from_checkpoint (Mat::stack over checkpoint names): a 16-bit in_ba-shaped matrix (96 rows) stays bf16 in a
    pre-quantized checkpoint and is requantized to int8 in a bf16 one, as the reference's int8 load mode does."""
    k, n = 1024, 96
    w = _weights(81, n, k)
    save_safetensors(str(tmp_path / "model.safetensors"), {"model.layers.0.linear_attn.in_proj_ba.weight": ("BF16", w)})
    cfg = {}
    if prequantized:
        cfg["quantization_config"] = {"format": "pack-quantized", "config_groups": {"group_0": {"weights": {
            "num_bits": 4, "type": "int", "strategy": "group", "group_size": 128, "symmetric": True}}}}
    (tmp_path / "config.json").write_text(json.dumps(cfg))
    ck = Checkpoint(str(tmp_path))
    mat = Mat.from_checkpoint(gemm, ck, ["model.layers.0.linear_attn.in_proj_ba.weight"], int8=True)
    assert mat.wt == (Wt.BF16 if prequantized else Wt.I8)
    x = activations(82, "x", 1, k)
    got = _plain(gemm, mat, x, 1)
    if prequantized:
        want = oracle.dense_f64(w, x)
    else:  # the product of the requantized weights (q - 128) s, per row and 128 columns
        vals, sc = oracle.requant_int8(w)
        wq = (vals.astype(np.float64) - 128.0) * np.repeat(sc.reshape(n, -1), 128, axis=1)
        want = bf16_to_f32(x).astype(np.float64) @ wq.T
    assert rel_err(got, want) <= 1e-4
