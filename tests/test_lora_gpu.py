"""Parity of the LoRA consumers (kernels/lora.cuh:52-113, launched by src/cuda/qwen/lora.rs:143-190) through the C ABI:
an unmerged adapter's delta s_t B (A x) added to a plain product's split 0 (lora_add), or the SwiGLU of a whole
[gate; up] product with the delta added first (lora_silu), for the tokens of the slots that use the adapter.

Against the oracle on random partials and B (f32 sums, f32 dot products in column order: 1e-5 of the output's RMS),
and end to end: the product's partials from an int4 matrix, xa from the stacked A product (a dense bf16 matrix),
lora_add, then sum_parts, against W x + s B (A x) in f64 (1e-4 of RMS, the int4 weights rounded to bf16 as the prefill
kernel does above 48 tokens); lora_silu against silu(g + dg) (u + du) with the bf16 rounding of the output.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat, lora_add, lora_silu, row_order, sum_parts
from qwenny_amd.synth import activations, bf16_to_f32, f32_to_bf16
from tests.helpers import bf16_out_err, emulate_bf16_weights, make_quant, oracle_y, rel_err, to_dev

pytestmark = pytest.mark.gpu
INT_MAX = 2**31 - 1


def _dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to("cuda") if dtype is None else t.view(dtype).to("cuda")


def _b16(b):
    import torch

    return _dev(np.ascontiguousarray(b, np.float16).view(np.int16), torch.int16)


@pytest.mark.parametrize("rank,split,n,m_cols,ends", [
    (8, 1, 1, 16, (64, 128)), (16, 3, 5, 48, (64, 128)), (32, 2, 13, 96, (64, 128)), (64, 4, 17, 256, (64, 128)),
    (16, 2, 40, 48, (72, 130)), (64, 1, 33, 256, (8, 184))])
def test_lora_add_matches_oracle(gemm, rank, split, n, m_cols, ends):
    """Module ends on tile boundaries (64, 128) and inside tiles (72, 130; 8, 184): a tile that straddles a module end
    takes each module's rows with that module's columns of xa; 33 and 40 tokens span two token workgroups."""
    import torch

    print(f"lora_add rank={rank} split={split} n={n} ends={ends}", flush=True)
    rng = np.random.default_rng(rank * 100 + n)
    rows = 192
    xa = rng.standard_normal((split, n, m_cols)).astype(np.float32)
    b = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float16)
    # three modules: rows 0..e0 from column 0, e0..e1 not adapted, e1..191 from the last rank columns
    e0, e1 = ends
    tab = np.array([e0, e1, INT_MAX, INT_MAX, 0, -1, m_cols - rank, -1], np.int32)
    slot_scale = np.array([0.0, 0.25, 2.0], np.float32)
    tok_slot = rng.integers(0, 3, n).astype(np.int32)
    y0 = rng.standard_normal((n, rows)).astype(np.float32)
    y = _dev(y0)
    lora_add(None, _dev(xa), split, m_cols, _b16(b), rank, rows, _dev(tab), _dev(tok_slot), _dev(slot_scale), n, y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = oracle.lora_add(y0, xa, split, b.view(np.uint16), rank, tab, tok_slot, slot_scale, n)
    assert rel_err(got, want) <= 1e-5
    untouched = slot_scale[tok_slot] == 0
    assert (got[untouched] == y0[untouched]).all()
    assert (got[:, e0:e1] == y0[:, e0:e1]).all()


@pytest.mark.parametrize("m", [1, 5, 40, 64, 200])
def test_lora_add_end_to_end(gemm, m):
    """y = W x + s B (A x): W int4 (1024 x 512) as plain split-K partials, xa = A x from a dense bf16 A of two rank-16
    modules (32 rows), the delta on split 0 of the product, then the partials summed. At 64 and 200 tokens both
    products are K-sliced prefill products (4 partials each)."""
    import torch

    print(f"lora_add end to end m={m}", flush=True)
    k, n_out, rank = 512, 1024, 16
    q = make_quant(150, "i4", n_out, k)
    w = Mat.stack(gemm, [q])
    rng = np.random.default_rng(151)
    a_bf16 = f32_to_bf16((rng.standard_normal((2 * rank, k)) * 0.05).astype(np.float32))
    amat = Mat.new(gemm, a_bf16, k, int8=False)
    b = (rng.standard_normal((n_out, rank)) * 0.05).astype(np.float16)
    tab = np.array([512, INT_MAX, INT_MAX, INT_MAX, 0, rank, -1, -1], np.int32)  # two modules of 512 rows
    slot_scale = np.array([0.0, 1.5], np.float32)
    tok_slot = (np.arange(m) % 2).astype(np.int32)
    x = activations(152, "x", m, k)
    xd = to_dev(x)
    split = w.split(m)
    y = torch.empty((split, m, n_out), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, w, xd, y, Epi.Plain) == split
    split_a = amat.split(m)
    xa = torch.empty((split_a, m, 2 * rank), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, amat, xd, xa, Epi.Plain) == split_a
    lora_add(None, xa, split_a, 2 * rank, _b16(b), rank, n_out, _dev(tab), _dev(tok_slot), _dev(slot_scale), m, y[0])
    out = torch.empty((m, n_out), dtype=torch.float32, device="cuda")
    sum_parts(None, y, split, m, n_out, out)
    torch.cuda.synchronize()
    ax = bf16_to_f32(x).astype(np.float64)
    xs = ax @ bf16_to_f32(a_bf16).astype(np.float64).T  # A x, [m][32]
    bf = b.astype(np.float64)
    delta = np.concatenate([xs[:, :rank] @ bf[:512].T, xs[:, rank:] @ bf[512:].T], axis=1)
    # decode products are exact; prefill ones round each int4 weight to bf16 once (the same bar on that arithmetic)
    base = oracle_y(q, x) if w.kernel(m) == "skinny" else emulate_bf16_weights(q, x)
    want = base + slot_scale[tok_slot][:, None] * delta
    assert rel_err(out.cpu().numpy(), want) <= 1e-4


@pytest.mark.parametrize("m", [5, 40])
def test_lora_silu_end_to_end(gemm, m):
    """mid = silu(gate + dg) (up + du): the whole [gate; up] product (split 1), the adapter on both modules."""
    import torch

    print(f"lora_silu end to end m={m}", flush=True)
    k, half, rank = 512, 256, 8
    gate, up = make_quant(160, "i4", half, k), make_quant(161, "i4", half, k)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    rows = 2 * half
    rng = np.random.default_rng(162)
    b_orig = (rng.standard_normal((rows, rank)) * 0.05).astype(np.float16)  # original [gate; up] order
    b = b_orig[row_order(rows, True)]  # the product's row order
    xa_host = rng.standard_normal((1, m, 16)).astype(np.float32)
    tab = np.array([INT_MAX] * 4 + [0, 8, -1, -1], np.int32)
    slot_scale = np.array([0.5, 0.0], np.float32)
    tok_slot = (np.arange(m) % 2).astype(np.int32)
    x = activations(163, "x", m, k)
    y = torch.empty((1, m, rows), dtype=torch.float32, device="cuda")
    assert gemm.run_split(None, m, mat, to_dev(x), y, Epi.Plain, True) == 1
    mid = torch.full((m, half), float("nan"), dtype=torch.bfloat16, device="cuda")
    lora_silu(None, _dev(xa_host), 1, 16, _b16(b), rank, rows, _dev(tab), _dev(tok_slot), _dev(slot_scale), m, y[0],
              mid)
    torch.cuda.synchronize()
    got = mid.float().cpu().numpy()
    packed = y[0].cpu().numpy()
    assert bf16_out_err(got, oracle.lora_silu(packed, xa_host, 1, b.view(np.uint16), rank, tab, tok_slot, slot_scale,
                                              m)) <= 1e-3
    # and against the math in the original order: gate + s B_g xa[0:8], up + s B_u xa[8:16]
    s = slot_scale[tok_slot].astype(np.float64)[:, None]
    xs = xa_host[0].astype(np.float64)
    full = np.concatenate([oracle_y(gate, x) + s * (xs[:, :8] @ b_orig[:half].astype(np.float64).T),
                           oracle_y(up, x) + s * (xs[:, 8:] @ b_orig[half:].astype(np.float64).T)], axis=1)
    assert bf16_out_err(got, oracle.silu_glu(full, None)) <= 2e-2


def test_lora_rejects(gemm):
    import torch

    from qwenny_amd._lib import QhError

    z = torch.zeros(1024, dtype=torch.float32, device="cuda")
    b = torch.zeros(1024, dtype=torch.int16, device="cuda")
    t = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(QhError):  # rank 12
        lora_add(None, z, 1, 16, b, 12, 16, t, t, z, 1, z)
    with pytest.raises(QhError):  # 512 columns of xa
        lora_add(None, z, 1, 512, b, 8, 16, t, t, z, 1, z)
    with pytest.raises(QhError):  # SwiGLU rows not in whole tiles
        lora_silu(None, z, 1, 16, b, 8, 24, t, t, z, 1, z, z)
    with pytest.raises(QhError):  # y rows not 16-byte aligned (ldy 18)
        lora_add(None, z, 1, 16, b, 8, 16, t, t, z, 1, z, ldy=18)
    with pytest.raises(QhError):  # y not 16-byte aligned
        lora_add(None, z, 1, 16, b, 8, 16, t, t, z, 1, z[1:])
    with pytest.raises(QhError):  # mid not 8-byte aligned
        lora_silu(None, z, 1, 16, b, 8, 16, t, t, z, 1, z, z.view(torch.int16)[1:])
