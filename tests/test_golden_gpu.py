"""The reference's own known-answer vectors through the HIP kernels: the affine int4 product cases of its kernel test
(src/mlx/metal.rs:369-428), committed as tests/golden/mlx_affine.npz by tests/golden/make_golden.py. Their scales are
f16 values (sc = f16((i % 11 + 1) / 97)) with offsets bi = -8 sc, i.e. symmetric int4 (zero point 8) whose scales
bf16 does not hold exactly, so the loader stores them as QH_WT_I4_S32 (f32 scales). The cases with 128-column groups
are served here (the reference's group-64 cases and its int8 case, with zero point 8 rather than 128, do not fit the
tile layout); output rows are padded to whole 16-row tiles with zero-weight rows. Every case is a decode-sized
product (1-8 tokens) on the skinny kernel, whose products are exact, so the reference test's own bar applies:
|got - want| < 2e-5 (1 + |want|) (src/mlx/metal.rs:404-406). The same generator at the 27B-scale shapes of the
reference's packed-layout test (src/mlx/metal.rs:430-485: [gate; up] 34816 x 5120, down 5120 x 17408, the 248,320-row
head, at 5 and 8 tokens) is held to that test's bar, max |got - want| < 2e-4."""

import os

import numpy as np
import pytest

from qwenny_amd import Epi, Mat, Wt
from qwenny_amd.core import Quant
from tests.helpers import to_dev

pytestmark = pytest.mark.gpu

PATH = os.path.join(os.path.dirname(__file__), "golden", "mlx_affine.npz")


def _cases():
    d = np.load(PATH)
    return [i for i in range(int(d["count"])) if int(d[f"bits{i}"]) == 4 and int(d[f"group{i}"]) % 128 == 0]


def test_golden_cases_present():
    assert len(_cases()) == 5


@pytest.mark.parametrize("i", _cases())
@pytest.mark.parametrize("whole", [False, True])
def test_mlx_affine_golden(gemm, i, whole):
    import torch

    d = np.load(PATH)
    m, n, k = (int(v) for v in d[f"shape{i}"])
    group = int(d[f"group{i}"])
    print(f"golden mlx affine case {i}: m={m} n={n} k={k} whole={whole}", flush=True)
    q, sc, bi = d[f"q{i}"], d[f"sc{i}"], d[f"bi{i}"]
    rows = (n + 15) // 16 * 16
    # padding rows: codes 8 (the zero point), so their weights are exactly zero
    qp = np.full((rows, q.shape[1]), 0x88888888, np.uint32)
    qp[:n] = q
    scp = np.full((rows, sc.shape[1]), sc.flat[0], np.float32)
    scp[:n] = sc
    bip = -8.0 * scp
    bip[:n] = bi
    quant = Quant(4, group, rows, k, qp, scp.reshape(-1), bip.reshape(-1))
    mat = Mat.stack(gemm, [quant])
    assert mat.wt == Wt.I4_S32
    assert mat.kernel(m, whole=whole) == "skinny"
    split = 1 if whole else mat.split(m)
    y = torch.full((split, m, rows), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run_split(None, m, mat, to_dev(d[f"xb{i}"]), y, Epi.Plain, whole) == split
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64).sum(0)
    want = d[f"y{i}"]
    assert (got[:, n:] == 0).all()
    err = np.abs(got[:, :n] - want)
    assert (err < 2e-5 * (1 + np.abs(want))).all(), err.max()


# the 27B-scale shapes of the reference's packed-layout test (src/mlx/metal.rs:436-444; (m, n, k), group 128):
# inputs from the same closed-form generator, expected products in f64 from the stored values, the test's own bar:
# max |got - want| < 2e-4 (src/mlx/metal.rs:478-480)
SHAPES_27B = [(5, 256, 1024), (8, 384, 5120), (5, 34816, 5120), (5, 5120, 17408), (5, 248320, 5120)]


@pytest.mark.parametrize("m,n,k", SHAPES_27B)
def test_mlx_affine_27b_shapes(gemm, m, n, k):
    import torch

    from tests.golden.make_golden import mlx_case
    from tests.test_full_output_gpu import _Dequant
    from qwenny_amd.synth import bf16_to_f32, f32_to_bf16

    print(f"golden generator 27B shape m={m} n={n} k={k}", flush=True)
    x16, q, sc, bi = mlx_case(m, n, k, 128, 4)
    quant = Quant(4, 128, n, k, q, sc.astype(np.float32).reshape(-1), bi.astype(np.float32).reshape(-1))
    mat = Mat.stack(gemm, [quant])
    assert mat.wt == Wt.I4_S32 and mat.kernel(m) == "skinny"
    xb = f32_to_bf16(x16.astype(np.float32))
    split = mat.split(m)
    y = torch.full((split, m, n), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(xb), y, Epi.Plain) == split
    torch.cuda.synchronize()
    got = y.double().sum(0).cpu().numpy()
    xf = bf16_to_f32(xb).astype(np.float64)
    dq = _Dequant(quant, 4096)
    worst = 0.0
    for r0 in range(0, n, 4096):
        r1 = min(n, r0 + 4096)
        worst = max(worst, float(np.abs(got[:, r0:r1] - xf @ dq.rows(r0, r1).T).max()))
    assert worst < 2e-4, worst
