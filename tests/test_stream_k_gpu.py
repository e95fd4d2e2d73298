"""Parity of the prefill kernel where the launcher spreads work items over the resident workgroups by groups of K
(stream-K): items cut between workgroups are summed from partials by the last workgroup to finish its segment.

The shapes are chosen so that the launcher's cost rule picks stream-K: (m, 4096, 4096) runs 96 items of 64 x 128 at
m = 130 and 64 of 128 x 128 at m = 256, fewer than one round at any occupancy of 1-8 workgroups per CU; (512, 17408,
5120) runs 136 items of 256 x 256 at the one workgroup per CU that shape holds. Same bar as the other prefill tests:
the oracle to 2e-2 RMS, and the kernel's own arithmetic (bf16-rounded weights, exact f64 sums) to 1e-4.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, row_order
from qwenny_amd.synth import activations
from tests.helpers import (TOL, bf16_out_err, emulate_bf16_weights, emulate_silu_prefill, make_quant, oracle_y, rel_err,
                           silu_bar, sub_quant, to_dev)

pytestmark = pytest.mark.gpu


def _run_plain(gemm, mat, x, m):
    import torch

    y = torch.full((1, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    # one partial (whole): short plain products otherwise take K-sliced partials instead of stream-K
    assert gemm.run_split(None, m, mat, to_dev(x), y, Epi.Plain, True) == 1
    torch.cuda.synchronize()
    return y[0].cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("kind", ["i4", "i4z", "i8", "i8g"])
@pytest.mark.parametrize("m", [130, 256])
def test_stream_k_plain(gemm, kind, m):
    print(f"stream-K plain {kind} m={m}", flush=True)
    n, k = 4096, 4096
    q = make_quant(71 + m, kind, n, k)
    mat = Mat.stack(gemm, [q])
    # twice with different activations: the item counters must be left at zero by each launch
    for rep in range(2):
        x = activations(80 + rep, "x", m, k, outliers=0.01)
        got = _run_plain(gemm, mat, x, m)
        assert rel_err(got, oracle_y(q, x)) <= TOL, rep
        assert rel_err(got, emulate_bf16_weights(q, x)) <= 1e-4, rep


def test_stream_k_27b_gate(gemm):
    """The 27B gate/up shape at a 512-token chunk, checked on a sample of 512 output rows over two launches."""
    print("stream-K 512 x 17408 x 5120", flush=True)
    n, k, m = 17408, 5120, 512
    q = make_quant(90, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    rows = np.sort(np.random.default_rng(5).choice(n, 512, replace=False))
    sq = sub_quant(q, rows)
    for rep in range(2):
        x = activations(91 + rep, "x", m, k, outliers=0.01)
        got = _run_plain(gemm, mat, x, m)[:, rows]
        assert not np.isnan(got).any()
        assert rel_err(got, oracle_y(sq, x)) <= TOL, rep
        assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4, rep


def test_stream_k_silu(gemm):
    """The SwiGLU epilogue on cut items: the summed partials feed silu(gate) * up."""
    import torch

    print("stream-K silu", flush=True)
    n, k, m = 4096, 4096, 256
    gate = make_quant(95, "i4", n // 2, k)
    up = make_quant(96, "i4", n // 2, k)
    x = activations(97, "x", m, k)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    y = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    full = np.concatenate([emulate_silu_prefill(gate, x), emulate_silu_prefill(up, x)], axis=1)
    want = oracle.silu_glu(full, row_order(n, True))
    got = y.float().cpu().numpy()
    assert bf16_out_err(got, want) <= 1e-3
    g, u = oracle_y(gate, x), oracle_y(up, x)
    assert silu_bar(got, g, u) <= 1.0
    assert bf16_out_err(got, oracle.silu_glu(np.concatenate([g, u], axis=1), None)) <= TOL


@pytest.mark.parametrize("kind", ["i4", "i4z", "i8", "i8g"])
@pytest.mark.parametrize("m", [49, 64, 130, 256, 512])
@pytest.mark.parametrize("n,k", [(6144, 5120), (5120, 17408)])
def test_k_sliced_plain(gemm, kind, m, n, k):
    """Short plain prefill products write K-sliced partials (whole items cut into 2-16 slices of K, slice s into
    y[s]) instead of stream-K: the returned split matches qh_mat_split, every partial is written, and their sum is the
    product (the oracle to 2e-2 RMS, the kernel's own arithmetic to 1e-4)."""
    import torch

    print(f"K-sliced plain {kind} m={m} {n}x{k}", flush=True)
    q = make_quant(180 + m, kind, n, k)
    mat = Mat.stack(gemm, [q])
    split = mat.split(m)
    rows = np.sort(np.random.default_rng(m).choice(n, 256, replace=False))
    sq = sub_quant(q, rows)
    for rep in range(2):
        x = activations(181 + rep, "x", m, k, outliers=0.01)
        y = torch.full((split, m, n), float("nan"), dtype=torch.float32, device="cuda")
        assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
        torch.cuda.synchronize()
        parts = y.cpu().numpy().astype(np.float64)
        assert not np.isnan(parts).any()
        got = parts.sum(0)[:, rows]
        assert rel_err(got, oracle_y(sq, x)) <= TOL, rep
        assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4, rep
