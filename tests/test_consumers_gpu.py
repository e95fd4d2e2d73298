"""The consumers of the plain products' split-K partials on the GPU through the C ABI: sum_parts (kernels/qwen.cu:
141-143) bit-exact, add_rmsnorm (kernels/qwen.cu:57-80) with the residual bit-exact and the normalised bf16 output within
one bf16 rounding of the f64 norm; and the decode residual step end to end, split-K product then add_rmsnorm."""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, add_rmsnorm, sum_parts
from qwenny_amd.synth import activations, bf16_to_f32
from tests.helpers import TOL, bf16_out_err, make_quant, oracle_y, to_dev

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("splits,n,ld", [(1, 1, 4), (10, 1, 5120), (34, 5, 5120), (3, 300, 1024)])
def test_sum_parts(splits, n, ld):
    import torch

    print(f"sum_parts {splits}x{n}x{ld}", flush=True)
    x = np.random.default_rng(splits + n).standard_normal((splits, n, ld)).astype(np.float32)
    y = torch.full((n, ld), float("nan"), dtype=torch.float32, device="cuda")
    sum_parts(None, _dev(x), splits, n, ld, y)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), oracle.sum_parts(x, splits))


@pytest.mark.parametrize("splits,n,hidden", [(1, 1, 2560), (10, 1, 5120), (34, 5, 5120), (1, 64, 1024), (3, 128, 5120),
                                              (2, 1, 20480)])
def test_add_rmsnorm(splits, n, hidden):
    import torch

    print(f"add_rmsnorm {splits}x{n}x{hidden}", flush=True)
    rng = np.random.default_rng(hidden + splits)
    h = rng.standard_normal((n, hidden)).astype(np.float32)
    x = (rng.standard_normal((splits, n, hidden)) * 0.3).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    hd, y = _dev(h), torch.empty((n, hidden), dtype=torch.bfloat16, device="cuda")
    add_rmsnorm(None, hd, _dev(x), splits, n, hidden, _dev(w), y, 1e-6)
    torch.cuda.synchronize()
    want_h, want_y = oracle.add_rmsnorm(h, x, splits, w, 1e-6)
    assert np.array_equal(hd.cpu().numpy(), want_h)
    assert bf16_out_err(y.float().cpu().numpy(), want_y) <= 1e-5


@pytest.mark.parametrize("m", [1, 5])
def test_residual_step_after_split_product(gemm, m):
    """A down-projection-shaped int4 product at decode sizes writes split-K partials; add_rmsnorm sums them into the
    residual and normalises, against the f64 product plus the residual, normalised."""
    import torch

    print(f"residual step m={m}", flush=True)
    hidden, k = 1024, 2048
    q = make_quant(61, "i4", hidden, k)
    mat = Mat.stack(gemm, [q])
    x = activations(62, "x", m, k)
    split = mat.split(m)
    part = torch.empty((split, m, hidden), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), part, Epi.Plain) == split
    rng = np.random.default_rng(63)
    h = rng.standard_normal((m, hidden)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, hidden).astype(np.float32)
    hd, y = _dev(h), torch.empty((m, hidden), dtype=torch.bfloat16, device="cuda")
    add_rmsnorm(None, hd, part, split, m, hidden, _dev(w), y, 1e-6)
    torch.cuda.synchronize()
    d = h.astype(np.float64) + oracle_y(q, x)
    want = w * d / np.sqrt(np.mean(d * d, axis=1, keepdims=True) + 1e-6)
    assert np.max(np.abs(hd.cpu().numpy() - d)) <= 1e-4 * np.sqrt(np.mean(d * d))
    assert bf16_out_err(y.float().cpu().numpy(), want) <= TOL
