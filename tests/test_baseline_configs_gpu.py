"""BASELINE.json's configurations at their full sizes on the GPU. Every product runs at its real shape; the outputs are
checked on a sample of rows against the oracle (the whole output would cost the f64 oracle minutes), and the 27B
head's argmax key against the argmax of its full logits. Bars as elsewhere: decode sizes are exact products (1e-4 of
RMS against the f64 oracle); prefill rounds each weight to bf16 once (1e-4 against that arithmetic, 2e-2 against the
oracle); per-channel int8 is exact at every size.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, Wt
from qwenny_amd.synth import activations
from tests.helpers import TOL, emulate_bf16_weights, make_quant, oracle_y, rel_err, sub_quant, to_dev

pytestmark = pytest.mark.gpu

SET_4B = [(2560, 4096), (4096, 2560), (2560, 1024), (2560, 9728), (2560, 9728), (9728, 2560)]
SET_27B = [(5120, 17408), (5120, 17408), (17408, 5120), (5120, 6144), (6144, 5120)]
PREFILL_27B = [(5120, 17408), (17408, 5120), (5120, 6144)]


def _plain(gemm, mat, x, m):
    import torch

    split = mat.split(m)
    y = torch.empty((split, m, mat.rows), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
    torch.cuda.synchronize()
    return y.sum(0).cpu().numpy().astype(np.float64)


def _sample(n, count, seed):
    return np.sort(np.random.default_rng(seed).choice(n, count, replace=False))


@pytest.mark.parametrize("m", [1, 2, 4, 5, 8])
def test_config1_4b_set_with_zero_points(gemm, m):
    print(f"configs[1] 4B set with zero points, m={m}", flush=True)
    for i, (k, n) in enumerate(SET_4B):
        q = make_quant(200 + i, "i4z", n, k)
        mat = Mat.stack(gemm, [q])
        assert mat.wt == Wt.I4Z
        x = activations(210 + i, "x", m, k)
        rows = _sample(n, 256, i)
        got = _plain(gemm, mat, x, m)[:, rows]
        assert rel_err(got, oracle_y(sub_quant(q, rows), x)) <= 1e-4, (k, n)


@pytest.mark.parametrize("m", [1, 5])
def test_config2_27b_set_and_head(gemm, m):
    import torch

    print(f"configs[2] 27B set and head, m={m}", flush=True)
    for i, (k, n) in enumerate(SET_27B):
        q = make_quant(300 + i, "i4", n, k)
        mat = Mat.stack(gemm, [q])
        x = activations(310 + i, "x", m, k)
        rows = _sample(n, 256, 10 + i)
        got = _plain(gemm, mat, x, m)[:, rows]
        assert rel_err(got, oracle_y(sub_quant(q, rows), x)) <= 1e-4, (k, n)
    k, n = 5120, 248320
    q = make_quant(320, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    x = activations(321, "x", m, k)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    keys = torch.zeros(m, dtype=torch.int64, device="cuda")
    gemm.run(None, m, mat, to_dev(x), y, Epi.Argmax, n_out=m, keys=keys)
    torch.cuda.synchronize()
    logits = y.cpu().numpy()
    assert (keys.cpu().numpy().view(np.uint64) == oracle.argmax_keys(logits, n)).all()
    want = oracle_y(q, x)  # all 248,320 rows, f64
    assert rel_err(logits, want) <= 1e-4
    assert (np.argmax(logits, axis=1) == np.argmax(want, axis=1)).all()


@pytest.mark.parametrize("m", [256, 512, 2048])
@pytest.mark.parametrize("kind", ["i4", "i4z"])
def test_config3_prefill(gemm, m, kind):
    print(f"configs[3] prefill {kind} m={m}", flush=True)
    for i, (k, n) in enumerate(PREFILL_27B):
        q = make_quant(400 + i, kind, n, k)
        mat = Mat.stack(gemm, [q])
        x = activations(410 + i, "x", m, k, outliers=0.01)
        rows = _sample(n, 64, 20 + i)
        sq = sub_quant(q, rows)
        got = _plain(gemm, mat, x, m)[:, rows]
        assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4, (k, n)
        assert rel_err(got, oracle_y(sq, x)) <= TOL, (k, n)


@pytest.mark.parametrize("m", [1, 5, 2048])
def test_config4_int8_per_channel(gemm, m):
    print(f"configs[4] int8 per channel m={m}", flush=True)
    for i, (k, n) in enumerate([(5120, 17408), (17408, 5120)]):
        q = make_quant(500 + i, "i8", n, k)
        mat = Mat.stack(gemm, [q])
        assert mat.wt == Wt.I8
        x = activations(510 + i, "x", m, k)
        rows = _sample(n, 64 if m > 16 else 256, 30 + i)
        got = _plain(gemm, mat, x, m)[:, rows]
        assert rel_err(got, oracle_y(sub_quant(q, rows), x)) <= 1e-4, (k, n)
