"""Pins of the CPU oracle (oracle/) against hand-built known answers, closed forms, library routines and the
reference's own known-answer generator — so that the oracle is checked against something other than itself."""

import numpy as np
import pytest

import oracle
from qwenny_amd.synth import bf16_to_f32, f32_to_bf16

# ---- Checkpoint::packed_matrix (src/checkpoint.rs:408-453) and Quant::row_into (:39-47) ---------------------------


def test_packed_matrix_symmetric_known_values():
    # one row of 16 int4 values 0..15: value c in word c / 8 at bits 4 (c % 8) (src/checkpoint.rs:26)
    words = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    scale = np.array([[0.5, 0.25]], np.float32)  # groups of 8 columns
    bits, group, cols, sc, off = oracle.packed_matrix(words, scale, 4, 8)
    assert (bits, group, cols) == (4, 8, 16)
    assert off.tolist() == [-4.0, -2.0]  # zero point 2^(bits-1) = 8
    row = oracle.row_into(bits, group, cols, words, sc, off, 0)
    want = [(c - 8) * 0.5 for c in range(8)] + [(c - 8) * 0.25 for c in range(8, 16)]
    assert row.tolist() == want


def test_packed_matrix_bits_from_shape():
    # 2 words for 8 columns: 8-bit values whatever the config says (src/checkpoint.rs:413)
    words = np.array([[0x04030201, 0x807F0000]], np.uint32)
    bits, group, cols, sc, off = oracle.packed_matrix(words, np.ones((1, 1), np.float32), 4, 0, cols=8)
    assert (bits, group, cols) == (8, 8, 8)
    row = oracle.row_into(bits, group, cols, words, sc, off, 0)
    assert row.tolist() == [1 - 128, 2 - 128, 3 - 128, 4 - 128, -128, -128, 127 - 128, 128 - 128]


def test_packed_matrix_zero_points_along_rows():
    # 9 rows, 2 groups: zero points packed 8 per word along the rows -> words [2][2]
    z = np.arange(18, dtype=np.uint32).reshape(9, 2) % 16
    zp = np.zeros((2, 2), np.uint32)
    for r in range(9):
        for g in range(2):
            zp[r // 8, g] |= z[r, g] << (4 * (r % 8))
    words = np.zeros((9, 2), np.uint32)
    scale = np.full((9, 2), 2.0, np.float32)
    _, _, _, sc, off = oracle.packed_matrix(words, scale, 4, 8, zero_point=zp)
    assert off.reshape(9, 2).tolist() == (-2.0 * z).tolist()


def test_packed_matrix_zero_points_along_groups():
    # 2 rows, 9 groups of 8: zero points packed along each row's groups -> words [2][2]
    z = (np.arange(18, dtype=np.uint32).reshape(2, 9) * 7) % 16
    zp = np.zeros((2, 2), np.uint32)
    for r in range(2):
        for g in range(9):
            zp[r, g // 8] |= z[r, g] << (4 * (g % 8))
    words = np.zeros((2, 9), np.uint32)
    _, _, _, sc, off = oracle.packed_matrix(words, np.ones((2, 9), np.float32), 4, 8, zero_point=zp)
    assert off.reshape(2, 9).tolist() == (-1.0 * z).tolist()


def test_packed_matrix_bad_zero_point_shape():
    with pytest.raises(ValueError):
        oracle.packed_matrix(np.zeros((4, 2), np.uint32), np.ones((4, 2), np.float32), 4, 8,
                             zero_point=np.zeros((3, 3), np.uint32))


# ---- Quant::zero_points (src/checkpoint.rs:72-82) -----------------------------------------------------------------


def test_zero_points():
    s = np.array([0.5, 0.25, 1e-3, 0.0], np.float32)
    assert oracle.zero_points(4, s, -8 * s).tolist() == [8, 8, 8, 0]  # s == 0 -> z 0
    assert oracle.zero_points(4, s[:3], -np.array([0, 15, 3], np.float32) * s[:3]).tolist() == [0, 15, 3]
    assert oracle.zero_points(4, s[:1], np.array([-8.2], np.float32) * s[:1]) is None  # not an integer
    assert oracle.zero_points(4, s[:1], np.array([-16.0], np.float32) * s[:1]) is None  # beyond 15
    assert oracle.zero_points(4, s[:1], np.array([1.0], np.float32) * s[:1]) is None  # negative
    near = np.array([-(3 + 5e-4)], np.float32) * s[:1]
    assert oracle.zero_points(4, s[:1], near).tolist() == [3]  # within 1e-3
    assert oracle.zero_points(8, np.ones(1, np.float32), np.array([-128.0], np.float32)).tolist() == [128]


# ---- row_order (src/cuda/core.rs:108-114) --------------------------------------------------------------------------


def test_row_order():
    want = list(range(0, 8)) + list(range(16, 24)) + list(range(8, 16)) + list(range(24, 32))
    assert oracle.row_order(32, True).tolist() == want
    assert oracle.row_order(32, False).tolist() == list(range(32))
    o = oracle.row_order(4096, True)
    assert sorted(o.tolist()) == list(range(4096))


# ---- int8 requantization (src/cuda/core.rs:356-369) ----------------------------------------------------------------


def test_requant_int8_known():
    w = np.zeros((2, 256), np.float32)
    w[0, 0] = 63.5  # max of group 0 -> scale 0.5
    w[0, 1] = 1.25  # 2.5 -> rounds half away from zero: 3
    w[0, 2] = -1.25  # -2.5 -> -3
    w[0, 3] = -63.5  # -127
    w[0, 4] = 0.75  # 1.5 -> 2
    w[1, 128] = -2.0  # group 1 of row 1: scale 2/127
    vals, sc = oracle.requant_int8(f32_to_bf16(w))
    assert sc[0, 0] == np.float32(63.5) / np.float32(127)
    assert sc[0, 1] == 1.0 and sc[1, 0] == 1.0  # all-zero groups
    assert sc[1, 1] == np.float32(2.0) / np.float32(127)
    q = vals.astype(int) - 128
    assert q[0, :5].tolist() == [127, 3, -3, -127, 2]
    assert (q[0, 5:] == 0).all() and q[1, 128] == -127
    assert vals.min() >= 1  # clamped to +-127, stored + 128


def test_requant_int8_roundtrip_error():
    rng = np.random.default_rng(0)
    w = f32_to_bf16(rng.standard_normal((16, 512)).astype(np.float32))
    vals, sc = oracle.requant_int8(w)
    deq = (vals.astype(np.float32) - 128) * np.repeat(sc, 128, axis=1)
    assert np.abs(deq - bf16_to_f32(w)).max() <= (np.repeat(sc, 128, axis=1) / 2 * 1.0001).max()


# ---- products: the f64 dequantize-then-matmul --------------------------------------------------------------------


def _rand_quant(seed, rows, cols, bits=4, group=128, zp=False):
    rng = np.random.default_rng(seed)
    words = rng.integers(0, 1 << 32, size=(rows, cols * bits // 32), dtype=np.uint32)
    sc = f32_to_bf16(rng.uniform(0.002, 0.02, (rows, cols // group)).astype(np.float32))
    z = None
    if zp:
        zz = rng.integers(0, 16, size=(rows, cols // group), dtype=np.uint32)
        z = np.zeros(((rows + 7) // 8, cols // group), np.uint32)
        for r in range(rows):
            z[r // 8] |= zz[r] << np.uint32(4 * (r % 8))
    b, g, c, s, o = oracle.packed_matrix(words, bf16_to_f32(sc), bits, group, zero_point=z)
    return b, g, c, words, s, o


def _dequant_numpy(bits, group, cols, words, s, o):
    """An independent dequantization with numpy vector ops (not the oracle's loop)."""
    per = 32 // bits
    shifts = (np.arange(cols) % per) * bits
    vals = (words[:, np.arange(cols) // per] >> shifts[None, :].astype(np.uint32)) & ((1 << bits) - 1)
    g = np.arange(cols) // group
    rows = words.shape[0]
    return vals * s.reshape(rows, -1)[:, g].astype(np.float64) + o.reshape(rows, -1)[:, g].astype(np.float64)


@pytest.mark.parametrize("bits,zp", [(4, False), (4, True), (8, False)])
def test_gemm_f64_matches_numpy(bits, zp):
    b, g, c, words, s, o = _rand_quant(1, 48, 512, bits, 128, zp)
    x = f32_to_bf16(np.random.default_rng(2).standard_normal((5, c)).astype(np.float32))
    y = oracle.gemm_f64(b, g, words, s, o, x)
    want = bf16_to_f32(x).astype(np.float64) @ _dequant_numpy(b, g, c, words, s, o).T
    assert np.abs(y - want).max() <= 1e-12 * np.abs(want).max()


def test_gemm_special_cases():
    b, g, c, words, s, o = _rand_quant(3, 32, 256)
    deq = _dequant_numpy(b, g, c, words, s, o)
    # one-hot x selects one column of the dequantized matrix
    x = np.zeros((1, c), np.float32)
    x[0, 77] = 1.0
    assert np.array_equal(oracle.gemm_f64(b, g, words, s, o, f32_to_bf16(x))[0], deq[:, 77])
    # every code equal to the zero point -> 0
    eight = np.full_like(words, 0x88888888)
    xr = f32_to_bf16(np.random.default_rng(4).standard_normal((3, c)).astype(np.float32))
    assert (oracle.gemm_f64(b, g, eight, s, o, xr) == 0).all()
    # s = 1, z = 0: exact integers
    ones, zeros = np.ones_like(s), np.zeros_like(o)
    xi = f32_to_bf16(np.random.default_rng(5).integers(-4, 5, (2, c)).astype(np.float32))
    y = oracle.gemm_f64(b, g, words, ones, zeros, xi)
    vals = _dequant_numpy(b, g, c, words, ones, zeros)
    assert np.array_equal(y, bf16_to_f32(xi).astype(np.float64) @ vals.T) and (y == np.round(y)).all()
    # linearity in x
    x1 = f32_to_bf16(np.random.default_rng(6).integers(-3, 4, (1, c)).astype(np.float32))
    x2 = f32_to_bf16(np.random.default_rng(7).integers(-3, 4, (1, c)).astype(np.float32))
    x12 = f32_to_bf16(bf16_to_f32(x1) + bf16_to_f32(x2))
    y1, y2, y12 = (oracle.gemm_f64(b, g, words, s, o, v) for v in (x1, x2, x12))
    assert np.allclose(y1 + y2, y12, rtol=1e-12, atol=1e-12)


def test_gemm_f32_close_to_f64():
    b, g, c, words, s, o = _rand_quant(8, 64, 1024)
    x = f32_to_bf16(np.random.default_rng(9).standard_normal((2, c)).astype(np.float32))
    y64 = oracle.gemm_f64(b, g, words, s, o, x)
    y32 = oracle.gemm_f32(b, g, words, s, o, x, threads=3)
    assert np.abs(y32 - y64).max() <= 1e-5 * np.sqrt((y64 ** 2).mean())


def test_mlx_known_answer_generator():
    """The reference's closed-form generator (src/mlx/metal.rs:375-384) and its tolerance 2e-5 (1 + |want|): the
    oracle reproduces the f64 loop of that test, recomputed here with numpy from the committed fixture's inputs."""
    from tests.golden.make_golden import mlx_case

    for m, n, k, group, bits in [(5, 64, 256, 128, 4), (1, 35, 1024, 128, 4), (8, 35, 256, 128, 8),
                                 (3, 35, 128, 64, 4)]:
        x16, q, sc, bi = mlx_case(m, n, k, group, bits)
        x = x16.astype(np.float32)
        # the oracle takes bf16 activations; use inputs exactly representable in both (the f16 values rounded)
        xb = f32_to_bf16(x)
        y = oracle.gemm_f64(bits, group, q, sc.astype(np.float32), bi.astype(np.float32), xb)
        want = bf16_to_f32(xb).astype(np.float64) @ _dequant_numpy(bits, group, k, q, sc.astype(np.float32),
                                                                    bi.astype(np.float32)).T
        assert (np.abs(y - want) < 2e-5 * (1 + np.abs(want))).all()


def test_golden_fixture():
    """The committed golden vectors (tests/golden/mlx_affine.npz, written by tests/golden/make_golden.py from the
    reference's generator) match the oracle."""
    import os

    path = os.path.join(os.path.dirname(__file__), "golden", "mlx_affine.npz")
    d = np.load(path)
    for i in range(int(d["count"])):
        bits, group = int(d[f"bits{i}"]), int(d[f"group{i}"])
        y = oracle.gemm_f64(bits, group, d[f"q{i}"], d[f"sc{i}"], d[f"bi{i}"], d[f"xb{i}"])
        want = d[f"y{i}"]
        assert (np.abs(y - want) < 2e-5 * (1 + np.abs(want))).all()


# ---- epilogues --------------------------------------------------------------------------------------------------


def test_silu_matches_torch():
    import torch

    y = np.random.default_rng(1).standard_normal((3, 64)) * 4
    got = oracle.silu_glu(y, None)
    t = torch.from_numpy(y)
    want = (torch.nn.functional.silu(t[:, :32]) * t[:, 32:]).numpy()
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_argmax_keys():
    lg = np.array([[1.0, 3.0, 3.0, -1.0], [-2.0, -1.0, -5.0, -1.0], [0.0, -0.0, 0.0, 7.0]], np.float32)
    keys = oracle.argmax_keys(lg, 3)  # row 2's 7.0 is past `valid`
    idx = 0xFFFFFFFF - (keys & 0xFFFFFFFF)
    assert idx.tolist() == [1, 1, 0]  # ties -> lowest index; -0.0 < +0.0 in the total order
    v = np.array([-np.inf, -3.0, -1e-30, -0.0, 0.0, 1e-30, 2.0, np.inf], np.float32)
    o = oracle.ordered(v)
    assert (np.diff(o.astype(np.int64)) > 0).all()


# ---- the dense 16-bit product (src/cuda/core.rs:370-381, kernels/gemm.cuh:120-212) ------------------------------


def test_dense_f64_closed_forms():
    """Small integers are exact in bf16, f16 and f64: the product is the integer matrix product, by hand; a one-hot x
    selects a weight column."""
    w = np.array([[1, -2, 3, 0], [4, 5, -6, 7]], np.float32)
    x = np.array([[2, 1, 0, -1], [0, 0, 1, 0]], np.float32)
    want = np.array([[0, 6], [3, -6]], np.float64)  # rows of x against rows of w
    for f16 in (False, True):
        assert np.array_equal(oracle.dense_f64(f32_to_bf16(w), f32_to_bf16(x), f16), want)


def test_dense_f64_f16_storage():
    """The reference's f16 storage changes a bf16 weight only outside f16's normal range: below 2^-14 it becomes an f16
    subnormal (a multiple of 2^-24, nearest even), above 65504 infinity; in range bf16 values are exact in f16."""
    w = f32_to_bf16(np.array([[1.0e-6], [3.140625], [-65536.0], [0.0078125]], np.float32))  # 4 rows, 1 column
    x = f32_to_bf16(np.ones((1, 1), np.float32))
    exact = oracle.dense_f64(w, x)[0]
    ref = oracle.dense_f64(w, x, f16_weights=True)[0]
    wf = bf16_to_f32(w)[:, 0]
    assert np.array_equal(exact, wf.astype(np.float64))
    assert ref[0] == round(float(wf[0]) / 2.0 ** -24) * 2.0 ** -24 and ref[0] != exact[0]
    assert ref[1] == exact[1] and ref[3] == exact[3]
    assert ref[2] == -np.inf


# ---- the trainer's dequant (kernels/qwen_train.cu:84-103) -------------------------------------------------------


def test_dequant_rows_known_words():
    """Hand-packed words: int4 values 0..15 along a row (low nibble first) with zero point 8 and scale 0.5; int8 bytes
    1, 0, 255, 128 with zero point 128 and scale 2. Every result is exact in bf16."""
    q4 = np.array([[0x76543210, 0xFEDCBA98] * 8], np.uint32)  # 128 columns: 0..15 repeated
    got = oracle.dequant_rows(4, 128, q4, np.array([0.5], np.float32), np.array([8], np.uint8), 0, 1)
    want = (np.tile(np.arange(16), 8) - 8) * 0.5
    assert np.array_equal(bf16_to_f32(got)[0], want.astype(np.float32))
    q8 = np.array([[0x80FF0001]], np.uint32)
    got = oracle.dequant_rows(8, 4, q8, np.array([2.0], np.float32), np.array([128], np.uint8), 0, 1, out_f32=True)
    assert np.array_equal(got[0], np.array([-254, -256, 254, 0], np.float32))


def test_dequant_rows_rounding_and_rows():
    """The f32 product rounds once, then to bf16 nearest even, checked against torch's bf16 conversion; rows r0..r0+n
    of the matrix and per-group scales and zero points."""
    import torch

    rng = np.random.default_rng(12)
    rows, cols, group = 6, 256, 128
    q = rng.integers(0, 2**32, (rows, cols // 8), dtype=np.uint64).astype(np.uint32)
    s = rng.uniform(0.001, 0.05, rows * 2).astype(np.float32)
    z = rng.integers(0, 16, rows * 2).astype(np.uint8)
    got32 = oracle.dequant_rows(4, group, q, s, z, 2, 3, out_f32=True)
    got16 = oracle.dequant_rows(4, group, q, s, z, 2, 3)
    for i, r in enumerate(range(2, 5)):
        for c in (0, 1, 127, 128, 255):
            v = (q[r, c // 8] >> (4 * (c % 8))) & 15
            w = np.float32(np.float32(int(v) - int(z[r * 2 + c // 128])) * s[r * 2 + c // 128])
            assert got32[i, c] == w
    want16 = torch.from_numpy(got32).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got16, want16)


# ---- the partials consumers (kernels/qwen.cu:57-80, :141-143) ----------------------------------------------------


def test_sum_parts_order_and_exactness():
    """Small integers sum exactly in any order; a large-magnitude case fixes the reference's order, (0 + x0) + x1 + x2:
    1e8 + 1 - 1e8 gives 0 in f32 (the 1 is lost), the other orders would not all agree."""
    x = np.array([[[1.0, 2.0]], [[3.0, -4.0]], [[5.0, 6.0]]], np.float32)
    assert np.array_equal(oracle.sum_parts(x, 3), np.array([[9.0, 4.0]], np.float32))
    y = np.array([[[1e8]], [[1.0]], [[-1e8]]], np.float32)
    assert oracle.sum_parts(y, 3)[0, 0] == 0.0
    assert oracle.sum_parts(y, 2)[0, 0] == np.float32(1e8)


def test_add_rmsnorm_closed_form():
    """h = (3, 4) with no partials: mean(h^2) = 12.5, so y = w h / sqrt(12.5 + eps); the partials add before the norm."""
    h = np.array([[3.0, 4.0]], np.float32)
    w = np.array([2.0, 0.5], np.float32)
    hn, y = oracle.add_rmsnorm(h, np.zeros((1, 1, 2), np.float32), 1, w, 1e-6)
    assert np.array_equal(hn, h)
    assert np.allclose(y, [[2 * 3 / np.sqrt(12.5 + 1e-6), 0.5 * 4 / np.sqrt(12.5 + 1e-6)]], rtol=1e-12)
    hn, y = oracle.add_rmsnorm(np.zeros((1, 2), np.float32), np.array([[[1.0, 2.0]], [[2.0, 2.0]]], np.float32), 2,
                               w, 0.0)
    assert np.array_equal(hn, h) and np.allclose(y, [[2 * 3 / np.sqrt(12.5), 0.5 * 4 / np.sqrt(12.5)]], rtol=1e-12)


# ---- LoRA consumers (kernels/lora.cuh) --------------------------------------------------------------------------


def _lora_case(seed, n=5, split=3, rank=8, m_cols=32):
    rng = np.random.default_rng(seed)
    xa = rng.standard_normal((split, n, m_cols)).astype(np.float32)
    slot_scale = np.array([0.0, 0.5, 2.0], np.float32)
    tok_slot = rng.integers(0, 3, n).astype(np.int32)
    return xa, slot_scale, tok_slot


def test_lora_add_one_hot_rows():
    """B[o] = e_(o % rank) makes the delta s_t * sum_s xa[s][t][off + o % rank]: a closed form."""
    n, split, rank, rows = 6, 3, 8, 32
    xa, slot_scale, tok_slot = _lora_case(1, n, split, rank)
    b = np.zeros((rows, rank), np.float16)
    b[np.arange(rows), np.arange(rows) % rank] = 1.0
    tab = [2**31 - 1] * 4 + [8, -1, -1, -1]
    y = np.random.default_rng(2).standard_normal((n, rows)).astype(np.float32)
    got = oracle.lora_add(y, xa, split, b.view(np.uint16), rank, tab, tok_slot, slot_scale, n)
    xs = xa.astype(np.float64).sum(0)
    want = y + slot_scale[tok_slot][:, None] * xs[:, 8 + np.arange(rows) % rank]
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    assert (got[slot_scale[tok_slot] == 0] == y[slot_scale[tok_slot] == 0]).all()


def test_lora_add_module_routing():
    """Three stacked modules (end rows 16, 48, 64): the first reads xa columns 0.., the second is not adapted, the third
    reads columns 8..; each equals the dense s * B_m (A x) of its own module."""
    n, split, rank = 4, 2, 8
    xa, slot_scale, tok_slot = _lora_case(3, n, split, rank, 16)
    rng = np.random.default_rng(4)
    b = rng.standard_normal((64, rank)).astype(np.float16)
    tab = [16, 48, 2**31 - 1, 2**31 - 1, 0, -1, 8, -1]
    y = np.zeros((n, 64), np.float32)
    got = oracle.lora_add(y, xa, split, b.view(np.uint16), rank, tab, tok_slot, slot_scale, n)
    xs = xa.astype(np.float64).sum(0)
    s = slot_scale[tok_slot].astype(np.float64)[:, None]
    assert np.allclose(got[:, :16], s * (xs[:, 0:8] @ b[:16].astype(np.float64).T))
    assert (got[:, 16:48] == 0).all()
    assert np.allclose(got[:, 48:], s * (xs[:, 8:16] @ b[48:].astype(np.float64).T))


def test_lora_silu_matches_swiglu_of_the_sum():
    """lora_silu = the SwiGLU epilogue (silu_glu over row_order's packing) of the plain product plus lora_add's delta."""
    from qwenny_amd import row_order

    n, split, rank, rows = 5, 2, 16, 64
    xa, slot_scale, tok_slot = _lora_case(5, n, split, rank, 32)
    rng = np.random.default_rng(6)
    b = rng.standard_normal((rows, rank)).astype(np.float16)  # rows in the packed (product) order
    tab = [2**31 - 1] * 4 + [0, 16, -1, -1]
    y = rng.standard_normal((n, rows)).astype(np.float32)  # packed order
    got = oracle.lora_silu(y, xa, split, b.view(np.uint16), rank, tab, tok_slot, slot_scale, n)
    # the same delta through lora_add, module 0 = packed gate rows, module 1 = packed up rows
    order = row_order(rows, True)  # packed row i <- original row order[i]
    gate_rows = np.flatnonzero(order < rows // 2)
    up_rows = np.flatnonzero(order >= rows // 2)
    full = np.zeros((n, rows), np.float64)
    for rows_m, off in ((gate_rows, 0), (up_rows, 16)):
        bm = np.zeros_like(b)
        bm[rows_m] = b[rows_m]
        t = [2**31 - 1] * 4 + [off, -1, -1, -1]
        full += oracle.lora_add(np.zeros_like(y), xa, split, bm.view(np.uint16), rank, t, tok_slot, slot_scale, n)
    orig = np.empty_like(full)
    orig[:, order] = y + full  # back to original order [gate; up]
    assert np.allclose(got, oracle.silu_glu(orig, None), rtol=1e-9, atol=1e-9)
