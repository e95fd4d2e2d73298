"""The LoRA delta fused into the product's epilogue (qh_gemm_lora), through the C ABI, against the oracle and against
the unfused path (the product, then the lora_add / lora_silu consumers, kernels/lora.cuh:52-113).

Plain products: the partials' sum must be W x + s_t B (A x) — the kernel's own product arithmetic (exact at decode
sizes, bf16-rounded weights above 48 tokens) plus the oracle's f64 delta, to 1e-4 of RMS — and the delta lands on
split 0 only (the other partials equal the plain product's). SwiGLU products: silu(gate + dg) (up + du) against the
oracle's lora_silu over the kernel's product (exact at decode sizes, f16 operands above 48 tokens), to one bf16 ulp
plus 1e-3 of RMS. Cases cover both kernels and every
prefill plan (K slices, stream-K, whole items), every rank, xa of 1-3 split-K partials, module ends inside tiles,
an unadapted module, and tokens of slot scale 0.
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import SKINNY_MAX_M, Epi, Mat, row_order
from qwenny_amd.synth import activations
from tests.helpers import bf16_out_err, emulate_bf16_weights, emulate_silu_prefill, make_quant, oracle_y, rel_err, to_dev

pytestmark = pytest.mark.gpu
INT_MAX = 2**31 - 1


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _adapter(rng, rows, rank, split, m, m_cols, tab):
    import torch

    xa = rng.standard_normal((split, m, m_cols)).astype(np.float32)
    b = (rng.standard_normal((rows, rank)) * 0.1).astype(np.float16)
    slot_scale = np.array([0.0, 0.5, 2.0], np.float32)
    tok_slot = rng.integers(0, 3, m).astype(np.int32)
    dev = (_dev(xa), split, m_cols, _dev(b.view(np.int16)), rank, _dev(np.asarray(tab, np.int32)), _dev(tok_slot),
           _dev(slot_scale))
    return dev, (xa, b.view(np.uint16), tab, tok_slot, slot_scale)


@pytest.mark.parametrize("m", [1, 5, 17, 48, 64, 130, 256, 512])
@pytest.mark.parametrize("rank,split,ends", [(8, 1, (256, 512)), (16, 2, (200, 712)), (64, 3, (8, 1000))])
def test_lora_plain_fused(gemm, m, rank, split, ends):
    import torch

    print(f"fused lora plain m={m} rank={rank} split={split} ends={ends}", flush=True)
    n, k = 1024, 2048
    q = make_quant(1400 + m, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    rng = np.random.default_rng(1401 + m + rank)
    m_cols = 2 * rank + 16
    e0, e1 = ends
    # module 0 from column 0, module 1 not adapted, module 2 from the last rank columns
    tab = [e0, e1, INT_MAX, INT_MAX, 0, -1, m_cols - rank, -1]
    dev, host = _adapter(rng, n, rank, split, m, m_cols, tab)
    x = activations(1402 + m, "x", m, k, outliers=0.01 if m > SKINNY_MAX_M else 0.0)
    xd = to_dev(x)
    sp = mat.split(m)
    y = torch.full((sp, m, n), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run_lora(None, m, mat, xd, y, Epi.Plain, dev) == sp
    y_plain = torch.full((sp, m, n), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, xd, y_plain, Epi.Plain) == sp
    torch.cuda.synchronize()
    got, plain = y.cpu().numpy(), y_plain.cpu().numpy()
    assert not np.isnan(got).any()
    # the delta on split 0 only; unadapted rows bit for bit the plain product's
    assert np.array_equal(got[1:], plain[1:])
    assert np.array_equal(got[0][:, e0:e1], plain[0][:, e0:e1])
    xa, b, tab_h, tok_slot, slot_scale = host
    base = oracle_y(q, x) if mat.kernel(m) == "skinny" else emulate_bf16_weights(q, x)
    want = oracle.lora_add(base, xa, split, b, rank, tab_h, tok_slot, slot_scale, m)
    assert rel_err(got.astype(np.float64).sum(0), want) <= 1e-4
    # against the unfused path on the same partials: the delta itself to f32 accuracy
    delta_got = got[0].astype(np.float64) - plain[0]
    delta_want = oracle.lora_add(np.zeros((m, n)), xa, split, b, rank, tab_h, tok_slot, slot_scale, m)
    assert rel_err(delta_got, delta_want) <= 1e-5 * max(1.0, float(np.sqrt(np.mean(plain[0] ** 2)) /
                                                            max(np.sqrt(np.mean(delta_want ** 2)), 1e-30)))


# split 1 with 16 or 32 columns of xa: prefill kernels stage the item's xa rows in LDS; (2048, 2048 + 2048, K 512):
# 256 x 256 items, the ping-pong schedule with the staged rows
@pytest.mark.parametrize("m,rank,split,half,k", [(m, r, s, 512, 1024) for m in (1, 5, 40, 64, 300) for r in (8, 32)
                                                 for s in (1, 2)] + [(2048, 16, 1, 2048, 512), (2048, 8, 2, 2048, 512)])
def test_lora_silu_fused(gemm, m, rank, split, half, k):
    import torch

    print(f"fused lora silu m={m} rank={rank} split={split} rows={2 * half} k={k}", flush=True)
    gate, up = make_quant(1500 + m, "i4", half, k), make_quant(1501 + m, "i4", half, k)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    rows = 2 * half
    rng = np.random.default_rng(1502 + m)
    m_cols = 2 * rank
    tab = [INT_MAX] * 4 + [0, rank, -1, -1]
    dev, host = _adapter(rng, rows, rank, split, m, m_cols, tab)
    x = activations(1503 + m, "x", m, k)
    mid = torch.full((m, half), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run_lora(None, m, mat, to_dev(x), mid, Epi.Silu, dev) == 1
    torch.cuda.synchronize()
    got = mid.float().cpu().numpy()
    order = row_order(rows, True)
    full = np.concatenate([oracle_y(gate, x), oracle_y(up, x)], axis=1) if mat.kernel(m, Epi.Silu) == "skinny" else \
        np.concatenate([emulate_silu_prefill(gate, x), emulate_silu_prefill(up, x)], axis=1)
    packed = full[:, order]  # the product in its packed (SwiGLU) row order
    xa, b, tab_h, tok_slot, slot_scale = host
    want = oracle.lora_silu(packed, xa, split, b, rank, tab_h, tok_slot, slot_scale, m)
    assert bf16_out_err(got, want) <= 1e-3


# Prefill products stage a one-split xa of 4-32 columns in LDS and read other forms from global memory: the same
# adapter given as one partial or as two (the second all zeros) must give the same outputs bit for bit (the sums run
# in the same order; 0 + p is p exactly). Plain (stream-K and whole items) and SwiGLU (the ping-pong 256 x 256 items).
@pytest.mark.parametrize("epi,m,half,k", [("plain", 256, 2048, 2048), ("plain", 2048, 2048, 512),
                                           ("silu", 2048, 2048, 512)])
def test_lora_staged_xa_matches_global(gemm, epi, m, half, k):
    import torch

    print(f"staged xa {epi} m={m} rows={2 * half} k={k}", flush=True)
    rank, rows = 16, 2 * half
    gate, up = make_quant(1700, "i4", half, k), make_quant(1701, "i4", half, k)
    mat = Mat.stack(gemm, [gate, up], silu=epi == "silu")
    rng = np.random.default_rng(1702)
    m_cols = 2 * rank
    tab = [half, INT_MAX, INT_MAX, INT_MAX, 0, rank, -1, -1]
    dev, host = _adapter(rng, rows, rank, 1, m, m_cols, tab)
    xa2 = torch.cat([dev[0], torch.zeros_like(dev[0])])  # the same xa as two partials
    dev2 = (xa2, 2) + dev[2:]
    x = to_dev(activations(1703, "x", m, k))
    outs = []
    for lora in (dev, dev2):
        if epi == "silu":
            y = torch.full((m, half), float("nan"), dtype=torch.bfloat16, device="cuda")
            assert gemm.run_lora(None, m, mat, x, y, Epi.Silu, lora) == 1
        else:
            sp = mat.split(m)
            y = torch.full((sp * m * rows,), float("nan"), dtype=torch.float32, device="cuda")
            assert gemm.run_lora(None, m, mat, x, y, Epi.Plain, lora) == sp
        torch.cuda.synchronize()
        outs.append(y.cpu())
    assert torch.equal(outs[0].view(torch.int16) if epi == "silu" else outs[0].view(torch.int32),
                       outs[1].view(torch.int16) if epi == "silu" else outs[1].view(torch.int32))


def test_lora_fused_rejects(gemm):
    import torch

    from qwenny_amd._lib import QhError

    mat = Mat.stack(gemm, [make_quant(1600, "i4", 64, 128)])
    z = torch.zeros(4096, dtype=torch.float32, device="cuda")
    t = torch.zeros(8, dtype=torch.int32, device="cuda")
    x = to_dev(activations(1, "x", 2, 128))
    with pytest.raises(QhError):  # rank 12
        gemm.run_lora(None, 2, mat, x, z, Epi.Plain, (z, 1, 16, z, 12, t, t, z))
    with pytest.raises(QhError):  # argmax takes no adapter
        gemm.run_lora(None, 2, mat, x, z, Epi.Argmax, (z, 1, 16, z, 8, t, t, z))
