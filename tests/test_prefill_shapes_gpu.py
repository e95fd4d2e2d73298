"""Parity of the 256 x 192 prefill workgroup shape (12 waves of 128 tokens x 32 outputs), which the launcher picks
over 256 x 256 when its whole rounds fill the CUs better: whole items at (2048 tokens, K 2048, 6144 outputs) through
the SwiGLU epilogue, and stream-K items at (512, 5120, 9216) through the plain one (a sample of rows). Same bars as the
other prefill tests: the oracle to 2e-2 RMS, the kernel's own arithmetic (bf16-rounded weights) to 1e-4, and the
SwiGLU output against silu over that arithmetic to 1e-3.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, row_order
from qwenny_amd.synth import activations
from tests.helpers import (TOL, bf16_out_err, emulate_bf16_weights, emulate_silu_prefill, make_quant, oracle_y, rel_err,
                           silu_bar, sub_quant, to_dev)

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["i4", "i4z", "i8", "i8g"])
def test_shape_256x192_stream_k_plain(gemm, kind):
    import torch

    print(f"prefill 256 x 192 stream-K plain {kind}", flush=True)
    n, k, m = 9216, 5120, 512
    q = make_quant(120, kind, n, k)
    mat = Mat.stack(gemm, [q])
    rows = np.sort(np.random.default_rng(6).choice(n, 384, replace=False))
    sq = sub_quant(q, rows)
    for rep in range(2):  # the item counters must be left at zero by each launch
        x = activations(121 + rep, "x", m, k, outliers=0.01)
        y = torch.full((1, m, n), float("nan"), dtype=torch.float32, device="cuda")
        # one partial (whole): the stream-K path, not the K-sliced partials of a short plain product
        assert gemm.run_split(None, m, mat, to_dev(x), y, Epi.Plain, True) == 1
        torch.cuda.synchronize()
        got = y[0].cpu().numpy().astype(np.float64)
        assert not np.isnan(got).any()
        got = got[:, rows]
        assert rel_err(got, oracle_y(sq, x)) <= TOL, rep
        assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4, rep


def test_shape_256x192_silu(gemm):
    import torch

    print("prefill 256 x 192 SwiGLU", flush=True)
    n, k, m = 6144, 2048, 2048
    gate = make_quant(130, "i4", n // 2, k)
    up = make_quant(131, "i4", n // 2, k)
    x = activations(132, "x", m, k, outliers=0.01)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    y = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    full = np.concatenate([emulate_silu_prefill(gate, x), emulate_silu_prefill(up, x)], axis=1)
    want = oracle.silu_glu(full, row_order(n, True))
    assert bf16_out_err(got, want) <= 1e-3
    g, u = oracle_y(gate, x), oracle_y(up, x)
    assert silu_bar(got, g, u) <= 1.0
    assert bf16_out_err(got, oracle.silu_glu(np.concatenate([g, u], axis=1), None)) <= TOL


def test_shape_256x192_dense_bf16(gemm):
    """Dense bf16 weights (the reference's Wt::F16) at the same stream-K shape: exact products, 1e-4 of RMS."""
    import torch

    from qwenny_amd.synth import f32_to_bf16

    print("prefill 256 x 192 stream-K dense bf16", flush=True)
    n, k, m = 9216, 5120, 512
    w = f32_to_bf16(np.random.default_rng(140).standard_normal((n, k)).astype(np.float32) * 0.05)
    mat = Mat.new(gemm, w, k, int8=False)
    x = activations(141, "x", m, k, outliers=0.01)
    y = torch.full((1, m, n), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run_split(None, m, mat, to_dev(x), y, Epi.Plain, True) == 1
    torch.cuda.synchronize()
    got = y[0].cpu().numpy().astype(np.float64)
    assert not np.isnan(got).any()
    rows = np.sort(np.random.default_rng(7).choice(n, 384, replace=False))
    assert rel_err(got[:, rows], oracle.dense_f64(w[rows], x)) <= 1e-4
