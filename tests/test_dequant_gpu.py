"""The trainer's dequant (kernels/qwen_train.cu:84-103) on the GPU through the C ABI, bit-exact against the oracle:
bf16 and f32 outputs, row ranges, int4 with and without zero points, int8 per channel, and rows whose word count is
not a multiple of 4 (the one-word path)."""

import numpy as np
import pytest

import oracle
from qwenny_amd import dequant
from tests.helpers import make_quant

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(kind, rows, cols, group):
    if kind in ("i4", "i4z", "i8"):
        q = make_quant(31, kind, rows, cols, group=group) if kind != "i8" else make_quant(31, kind, rows, cols)
        z = q.zero_points()
        assert z is not None
        return q.bits, q.group, q.q, q.scales, z
    # small odd shapes: random words, scales and zero points
    bits = 4 if kind == "odd4" else 8
    rng = np.random.default_rng(9)
    words = cols * bits // 32
    q = rng.integers(0, 2**32, (rows, words), dtype=np.uint64).astype(np.uint32)
    g = cols // group
    s = rng.uniform(0.001, 0.05, rows * g).astype(np.float32)
    z = rng.integers(0, 1 << bits, rows * g).astype(np.uint8)
    return bits, group, q, s, z


@pytest.mark.parametrize("kind,rows,cols,group", [("i4", 64, 1024, 128), ("i4z", 48, 512, 128),
                                                  ("i8", 32, 768, 768), ("odd4", 16, 136, 8), ("odd8", 16, 20, 4)])
@pytest.mark.parametrize("out_f32", [False, True])
def test_dequant_matches_oracle(kind, rows, cols, group, out_f32):
    import torch

    print(f"dequant {kind} {rows}x{cols} g{group} f32={out_f32}", flush=True)
    bits, group, q, s, z = _case(kind, rows, cols, group)
    words = q.shape[1]
    for r0, n in ((0, rows), (3, rows // 2), (rows - 1, 1)):
        out = torch.full((n, cols), -1, dtype=torch.float32 if out_f32 else torch.int16, device="cuda")
        dequant(None, _dev(q), _dev(s), _dev(z), rows, words, cols, group, bits, r0, n, out, out_f32)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = oracle.dequant_rows(bits, group, q, s, z, r0, n, out_f32)
        if out_f32:
            assert np.array_equal(got, want), (r0, n)
        else:
            assert np.array_equal(got.view(np.uint16), want), (r0, n)


def test_dequant_rejects():
    import torch

    from qwenny_amd._lib import QhError

    q = _dev(np.zeros((16, 16), np.uint32))
    s, z = _dev(np.ones(16, np.float32)), _dev(np.zeros(16, np.uint8))
    out = torch.empty((16, 128), dtype=torch.int16, device="cuda")
    with pytest.raises(QhError):  # rows past the matrix
        dequant(None, q, s, z, 16, 16, 128, 128, 4, 10, 7, out)
    with pytest.raises(QhError):  # words that do not hold the columns
        dequant(None, q, s, z, 16, 16, 120, 120, 4, 0, 1, out)
    with pytest.raises(QhError):  # 2-bit values
        dequant(None, q, s, z, 16, 16, 256, 128, 2, 0, 1, out)
