"""Parity of the products over the matrix forms the loader makes beyond a plain stored matrix: rows written later
(Mat::marlin_rows + Gemm::put_block, src/cuda/core.rs:140-153, :619-657), groups wider than 128 and one group per row,
f32 scales, strided activations, whole (unsplit) products, and a checkpoint read from disk end to end."""

import json

import numpy as np
import pytest

import oracle
from qwenny_amd import SKINNY_MAX_M, Epi, Mat, Quant, Wt, synth
from qwenny_amd.checkpoint import Checkpoint, save_safetensors
from qwenny_amd.synth import activations
from tests.helpers import TOL, make_quant, oracle_y, rel_err, sub_quant, to_dev

pytestmark = pytest.mark.gpu


def _plain(gemm, mat, x, m, whole=False, ldx=0, xdev=None):
    import torch

    split = 1 if whole else mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    got = gemm.run_split(None, m, mat, to_dev(x) if xdev is None else xdev, y, Epi.Plain, whole, ldx=ldx)
    torch.cuda.synchronize()
    assert got == split
    return y.sum(0).cpu().numpy().astype(np.float64)


def _argmax(gemm, mat, x):
    import torch

    m = x.shape[0]
    y = torch.zeros((m, mat.rows), dtype=torch.float32, device="cuda")
    keys = torch.zeros(m, dtype=torch.int64, device="cuda")
    gemm.run(None, m, mat, to_dev(x), y, Epi.Argmax, n_out=m, keys=keys)
    torch.cuda.synchronize()
    return y.cpu().numpy(), keys.cpu().numpy().view(np.uint64)


@pytest.mark.parametrize("kind", ["i4", "i4z"])
@pytest.mark.parametrize("m", [1, 5, 64])
def test_marlin_rows_then_put_block(gemm, kind, m):
    """A draft head: 32 rows uploaded in a matrix of room for 128, two blocks written later. The outputs of the
    written rows match the oracle on those stored rows; the argmax counts only the valid rows."""
    print(f"marlin_rows/put_block {kind} m={m}", flush=True)
    n, k = 256, 512
    q = make_quant(71, kind, n, k)
    zeros = q.zero_points()
    rng = np.random.default_rng(5)
    first = rng.choice(n, 32, replace=False)
    mat = Mat.marlin_rows(gemm, q, zeros, first, 128)
    assert (mat.rows, mat.valid, mat.wt) == (128, 32, Wt.I4Z if kind == "i4z" else Wt.I4)
    x = activations(9 + m, "x", m, k)
    got = _plain(gemm, mat, x, m)
    tol = 1e-4 if mat.kernel(m) == "skinny" else TOL
    assert rel_err(got[:, :32], oracle_y(sub_quant(q, first), x)) <= tol
    logits, keys = _argmax(gemm, mat, x)
    assert (keys == oracle.argmax_keys(logits, 32)).all()

    written = {}
    for block in (3, 5):
        rows = rng.choice(n, 16, replace=False)
        gemm.put_block(None, mat, q, zeros, block, rows)
        written[block] = rows
    assert mat.valid == 96
    got = _plain(gemm, mat, x, m)
    assert rel_err(got[:, :32], oracle_y(sub_quant(q, first), x)) <= tol
    for block, rows in written.items():
        assert rel_err(got[:, block * 16:(block + 1) * 16], oracle_y(sub_quant(q, rows), x)) <= tol
    logits, keys = _argmax(gemm, mat, x)
    assert (keys == oracle.argmax_keys(logits, 96)).all()


def test_put_block_rejects(gemm):
    from qwenny_amd._lib import QhError

    q = make_quant(72, "i4z", 64, 256)
    zeros = q.zero_points()
    sym = make_quant(73, "i4", 64, 256)
    mat = Mat.marlin_rows(gemm, sym, sym.zero_points(), np.arange(16), 64)
    assert mat.wt == Wt.I4
    if (zeros != 8).any():
        with pytest.raises(QhError):  # zero points into a symmetric matrix
            gemm.put_block(None, mat, q, zeros, 1, np.arange(16))
    with pytest.raises(QhError):  # block beyond the matrix
        gemm.put_block(None, mat, sym, sym.zero_points(), 4, np.arange(16))
    with pytest.raises(ValueError):
        gemm.put_block(None, mat, sym, sym.zero_points(), 1, np.arange(8))


@pytest.mark.parametrize("group", [256, 1024])
@pytest.mark.parametrize("m", [1, 3, 100])
def test_wide_groups(gemm, group, m):
    """Groups of 256 columns and one group per row (group = cols) are stored replicated per 128 columns."""
    print(f"group {group} m={m}", flush=True)
    q = make_quant(74, "i4z", 256, 1024, group=group)
    assert q.group == group
    x = activations(11, "x", m, 1024)
    mat = Mat.stack(gemm, [q])
    got = _plain(gemm, mat, x, m)
    assert rel_err(got, oracle_y(q, x)) <= (1e-4 if mat.kernel(m) == "skinny" else TOL)


@pytest.mark.parametrize("zp", [False, True])
@pytest.mark.parametrize("m", [1, 7, 40])
def test_f32_scales(gemm, zp, m):
    """Scales that bf16 does not hold (an f16 or f32 checkpoint) select the f32-scale storage, exact again."""
    print(f"f32 scales zp={zp} m={m}", flush=True)
    q = make_quant(75, "i4z" if zp else "i4", 128, 512)
    sc = (q.scales * (1 + np.random.default_rng(1).uniform(1e-3, 2e-3, q.scales.shape))).astype(np.float32)
    z = q.zero_points()
    off = (-z.astype(np.float32) * sc).astype(np.float32)
    q2 = Quant(q.bits, q.group, q.rows, q.cols, q.q, sc, off)
    mat = Mat.stack(gemm, [q2])
    assert mat.wt == (Wt.I4Z_S32 if zp else Wt.I4_S32)
    x = activations(12, "x", m, 512)
    assert rel_err(_plain(gemm, mat, x, m), oracle_y(q2, x)) <= (1e-4 if mat.kernel(m) == "skinny" else TOL)


@pytest.mark.parametrize("m", [1, 4, 33])
def test_strided_activations(gemm, m):
    """x rows with a leading dimension beyond the matrix's columns (a view into a wider buffer)."""
    import torch

    k, ldx = 512, 640
    q = make_quant(76, "i4", 128, k)
    wide = activations(13, "x", m, ldx)
    x = wide[:, :k]
    xdev = torch.from_numpy(np.ascontiguousarray(wide).view(np.int16)).cuda().view(torch.bfloat16)
    mat = Mat.stack(gemm, [q])
    got = _plain(gemm, mat, x, m, ldx=ldx, xdev=xdev)
    assert rel_err(got, oracle_y(q, np.ascontiguousarray(x))) <= (1e-4 if mat.kernel(m) == "skinny" else TOL)


@pytest.mark.parametrize("kind", ["i4", "i8"])
@pytest.mark.parametrize("m", [1, 6])
def test_whole(gemm, kind, m):
    """run_split(whole): one partial, the same values as the split product."""
    q = make_quant(77, kind, 256, 2048)
    x = activations(14, "x", m, 2048)
    mat = Mat.stack(gemm, [q])
    whole = _plain(gemm, mat, x, m, whole=True)
    assert rel_err(whole, oracle_y(q, x)) <= 1e-4
    assert rel_err(whole, _plain(gemm, mat, x, m)) <= 1e-5


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("kind,k", [("i4", 17408), ("i4z", 17408), ("i4", 9216), ("i4z", 2560)])
def test_whole_decode_long_k(gemm, kind, k, m):
    """run_split(whole) at 1-8 tokens on the workgroup-per-tile-pair kernels, whose waves take one or several chunks
    of 4 groups of K (17408: 34 chunks over 12 waves, 10 of them taking 3; 9216: 18 over 9): every row against the
    oracle, and the split product's value. 35 tiles: the last tile pair is half empty."""
    print(f"whole decode {kind} k={k} m={m}", flush=True)
    q = make_quant(79, kind, 560, k)
    x = activations(15 + m, "x", m, k)
    mat = Mat.stack(gemm, [q])
    whole = _plain(gemm, mat, x, m, whole=True)
    assert rel_err(whole, oracle_y(q, x)) <= 1e-4
    assert rel_err(whole, _plain(gemm, mat, x, m)) <= 1e-5


def test_part_len(gemm):
    mats = [Mat.stack(gemm, [make_quant(78, "i4", 256, k)]) for k in (512, 4096)]
    for max_tok in (16, SKINNY_MAX_M, SKINNY_MAX_M + 1, 300, 600):
        need = max(m.split(n) * n * m.rows for m in mats for n in range(1, max_tok + 1))
        assert gemm.part_len(mats, max_tok) >= need, max_tok
    # decode sizes: one partial per 4 groups of K; short prefill: up to 16 K slices; from 513 tokens: one
    assert mats[1].split(SKINNY_MAX_M) > 4 and 1 <= mats[1].split(SKINNY_MAX_M + 1) <= 16 and mats[1].split(513) == 1


def test_split_by_token_count(gemm):
    """A matrix whose 4-group waves would number too few per CU takes one group per wave (split = groups of K) at 1-2
    tokens and 4 groups from 3 (split = chunks); part_len covers both. configs[0]'s (2560, 9728): 304 wave columns x 5
    chunks = 1520 waves, below 6 per CU at one token, not below 4 from 3 tokens."""
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    q = make_quant(79, "i4", 9728, 2560)
    mat = Mat.stack(gemm, [q])
    waves = 304 * 5
    want = [20 if waves < (6 if n <= 2 else 4) * cus else 5 for n in (1, 2, 3, 5)]
    assert [mat.split(n) for n in (1, 2, 3, 5)] == want
    assert gemm.part_len([mat], 8) >= max(mat.split(n) * n * mat.rows for n in range(1, 9))


def test_checkpoint_end_to_end(gemm, tmp_path):
    """A compressed-tensors checkpoint on disk (gate with zero points, up and down symmetric) through Checkpoint,
    Quant.stack and Mat.stack into the SwiGLU product and the plain product after it."""
    import torch

    k, n = 512, 256
    gate = synth.int4_quant(81, "gate", n, k, zp=True)
    up = synth.int4_quant(82, "up", n, k)
    down = synth.int4_quant(83, "down", k, n)
    tensors = {}
    for name, t in (("gate_proj", gate), ("up_proj", up), ("down_proj", down)):
        p = f"model.layers.0.mlp.{name}"
        tensors[f"{p}.weight_packed"] = ("I32", t["weight_packed"].view(np.int32))
        tensors[f"{p}.weight_scale"] = ("BF16", t["weight_scale"])
        tensors[f"{p}.weight_shape"] = ("I64", t["weight_shape"])
        if "weight_zero_point" in t:
            tensors[f"{p}.weight_zero_point"] = ("I32", t["weight_zero_point"].view(np.int32))
    save_safetensors(str(tmp_path / "model.safetensors"), tensors)
    qc = {"format": "pack-quantized", "config_groups": {"group_0": {"weights": {
        "num_bits": 4, "type": "int", "strategy": "group", "group_size": 128, "symmetric": True}}}}
    (tmp_path / "config.json").write_text(json.dumps({"quantization_config": qc}))
    ck = Checkpoint(str(tmp_path))
    qg, qu, qd = (ck.quant_matrix(f"model.layers.0.mlp.{p}") for p in ("gate_proj", "up_proj", "down_proj"))
    gu = Mat.stack(gemm, [qg, qu], silu=True)
    dn = Mat.stack(gemm, [qd])
    assert (gu.wt, dn.wt) == (Wt.I4Z, Wt.I4)
    x = activations(15, "x", 2, k)
    h = torch.empty((2, n), dtype=torch.bfloat16, device="cuda")
    gemm.run(None, 2, gu, to_dev(x), h, Epi.Silu)
    torch.cuda.synchronize()
    full = np.concatenate([oracle_y(qg, x), oracle_y(qu, x)], axis=1)
    want_h = oracle.silu_glu(full, oracle.row_order(2 * n, True))
    assert rel_err(h.float().cpu().numpy(), want_h) <= TOL
    hb = h.view(torch.int16).cpu().numpy().view(np.uint16)
    got = _plain(gemm, dn, hb, 2)
    assert rel_err(got, oracle_y(qd, hb)) <= 1e-4
