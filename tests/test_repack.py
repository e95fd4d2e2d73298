"""The load-time repacker and the host-side weight formats of libqwenny_hip (no GPU): bit-exact round trips through the
gfx950 tile layout, and the product's host functions against the oracle."""

import numpy as np
import pytest

import oracle
from qwenny_amd import Wt, pack_dense_bf16, pack_dense_int8, pack_quant, packed_sizes, row_order, unpack_rows, \
    unpack_rows_bf16
from qwenny_amd.checkpoint import quant_from_packed
from qwenny_amd.core import Quant
from qwenny_amd.synth import bf16_to_f32, f32_to_bf16
from tests.helpers import make_quant


def stored_values(q):
    """The stored values [rows][cols] of a Quant, vectorised independently of the library."""
    per = 32 // q.bits
    c = np.arange(q.cols)
    return ((q.q[:, c // per] >> ((c % per) * q.bits).astype(np.uint32)) & ((1 << q.bits) - 1)).astype(np.uint8)


def per128(a, q):
    """[rows][cols / group] -> [rows][cols / 128] (a stored group of several 128-column groups replicated)."""
    return np.repeat(a.reshape(q.rows, -1), q.group // 128, axis=1)


@pytest.mark.parametrize("kind,silu", [("i4", False), ("i4", True), ("i4z", False), ("i4z", True), ("i8", False),
                                       ("i8", True)])
def test_roundtrip(kind, silu):
    q = make_quant(3, kind, 256, 640)
    z = q.zero_points()
    wt = {"i4": Wt.I4, "i4z": Wt.I4Z, "i8": Wt.I8}[kind]
    order = row_order(q.rows, silu)
    codes, scales, zeros = pack_quant(q, order, wt, z if wt.has_zeros else None)
    vals, sc, zz = unpack_rows(wt, q.rows, q.cols, codes, scales, zeros)
    assert np.array_equal(vals, stored_values(q)[order])
    assert np.array_equal(sc, per128(q.scales, q)[order])
    assert np.array_equal(zz, per128(z, q)[order])


def test_roundtrip_large_groups_and_f32_scales():
    # group 256 (two 128-column groups per stored scale) and scales bf16 does not hold: the f32-scale storage
    rng = np.random.default_rng(5)
    rows, cols = 64, 1024
    words = rng.integers(0, 1 << 32, size=(rows, cols // 8), dtype=np.uint32)
    scale = rng.uniform(0.002, 0.02, (rows, cols // 256)).astype(np.float32)  # not bf16-exact
    q = quant_from_packed(words, scale, 4, 256)
    z = q.zero_points()
    codes, scales, zeros = pack_quant(q, np.arange(rows), Wt.I4_S32)
    vals, sc, zz = unpack_rows(Wt.I4_S32, rows, cols, codes, scales, zeros)
    assert np.array_equal(vals, stored_values(q))
    assert np.array_equal(sc, per128(q.scales, q)) and (zz == 8).all() and (z == 8).all()


def test_roundtrip_rows_subset_and_padding():
    # marlin_rows: chosen rows then the first row repeated up to the capacity
    q = make_quant(4, "i4z", 128, 256)
    z = q.zero_points()
    rows = np.array([5, 77, 3, 120, 0, 1, 2, 9, 10, 11, 12, 13, 14, 15, 16, 17])
    order = np.concatenate([rows, np.full(16, rows[0])])
    codes, scales, zeros = pack_quant(q, order, Wt.I4Z, z)
    vals, sc, zz = unpack_rows(Wt.I4Z, 32, q.cols, codes, scales, zeros)
    assert np.array_equal(vals, stored_values(q)[order])
    assert np.array_equal(zz, per128(z, q)[order])


def test_layout_nibble_order():
    """The documented in-word order: column c at nibble c / 2 (even c) or 4 + c / 2 (odd c), so that the and-or with
    0x000F000F yields columns (2p, 2p + 1) in the (low, high) bf16 halves."""
    cols = 128
    words = np.zeros((16, cols // 8), np.uint32)
    for c in range(8):
        words[0, 0] |= np.uint32(c + 1) << np.uint32(4 * c)  # row 0, columns 0..7 hold 1..8
    q = quant_from_packed(words, np.ones((16, 1), np.float32), 4, 128)
    codes, _, _ = pack_quant(q, np.arange(16), Wt.I4)
    w = codes.view(np.uint32)[0]  # lane 0, step 0: row 0, columns 0..7
    for p in range(4):
        pair = (int(w) >> (4 * p)) & 0x000F000F
        assert (pair & 0xF, pair >> 16) == (2 * p + 1, 2 * p + 2)


def test_dense_int8_matches_oracle():
    rng = np.random.default_rng(6)
    w = f32_to_bf16(rng.standard_normal((48, 384)).astype(np.float32))
    w[3, 5] = 0  # and an all-zero group
    w[7, :128] = 0
    order = row_order(48, True)
    codes, scales = pack_dense_int8(w, order)
    vals, sc, zz = unpack_rows(Wt.I8, 48, 384, codes, scales)
    ovals, osc = oracle.requant_int8(w)
    assert np.array_equal(vals, ovals[order]) and np.array_equal(sc, osc[order]) and (zz == 128).all()


@pytest.mark.parametrize("silu", [False, True])
def test_dense_bf16_roundtrip(silu):
    """Dense 16-bit matrices keep their bf16 values bit for bit through the tile layout, in row_order."""
    w = f32_to_bf16(np.random.default_rng(8).standard_normal((96, 384)).astype(np.float32))
    order = row_order(96, silu)
    codes = pack_dense_bf16(w, order)
    assert codes.size == packed_sizes(Wt.BF16, 96, 384)[0] == 96 * 384 * 2
    assert packed_sizes(Wt.BF16, 96, 384)[1:] == (0, 0)
    assert np.array_equal(unpack_rows_bf16(96, 384, codes), w[order])


def test_dense_bf16_layout():
    """The documented block order: block (tile, group) = [step j][lane] 16 bytes, lane l holding row l % 16 and
    columns 32 j + 8 (l / 16) + 0..7 of the group, so each piece is a B fragment as loaded."""
    rows, cols = 32, 256
    w = np.arange(rows * cols, dtype=np.uint16).reshape(rows, cols)  # value = 256 row + column
    pieces = pack_dense_bf16(w, np.arange(rows)).view(np.uint16).reshape(rows // 16, cols // 128, 4, 64, 8)
    for t, g, j, l in [(0, 0, 0, 0), (0, 0, 0, 17), (0, 1, 3, 63), (1, 1, 2, 5)]:
        r, c0 = 16 * t + l % 16, 128 * g + 32 * j + 8 * (l // 16)
        assert np.array_equal(pieces[t, g, j, l], w[r, c0:c0 + 8])


# ---- the product's host functions vs the oracle -----------------------------------------------------------------


@pytest.mark.parametrize("zp", [False, True])
def test_quant_from_packed_matches_oracle(zp):
    from qwenny_amd import synth

    t = synth.int4_quant(9, "m", 40, 512, zp=zp)
    sc = bf16_to_f32(t["weight_scale"])
    q = quant_from_packed(t["weight_packed"], sc, 4, 128, t.get("weight_zero_point"), t["weight_shape"])
    b, g, c, osc, ooff = oracle.packed_matrix(t["weight_packed"], sc, 4, 128, zero_point=t.get("weight_zero_point"))
    assert (q.bits, q.group, q.cols) == (b, g, c)
    assert np.array_equal(q.scales, osc) and np.array_equal(q.offsets, ooff)
    for r in (0, 17, 39):
        assert np.array_equal(q.row_into(r), oracle.row_into(b, g, c, q.q, osc, ooff, r))
    zq, zo = q.zero_points(), oracle.zero_points(4, osc, ooff)
    assert np.array_equal(zq, zo)


def test_zero_points_non_integer():
    q = make_quant(1, "i4", 16, 128)
    q.offsets[3] += q.scales[3] * 0.01
    assert q.zero_points() is None


def test_row_order_matches_oracle():
    for rows in (16, 48, 4096):
        for silu in (False, True):
            assert np.array_equal(row_order(rows, silu), oracle.row_order(rows, silu))


@pytest.mark.parametrize("kind,rows", [("i4z", 16), ("i4", 97 * 16), ("i8", 40)])
def test_to_bf16(kind, rows):
    """Quant::to_bf16 (threaded over rows) against torch's nearest-even rounding of each row_into row."""
    import torch

    q = make_quant(2, kind, rows, 256)
    b = q.to_bf16()
    want = torch.from_numpy(np.stack([q.row_into(r) for r in range(rows)])).to(torch.bfloat16).view(torch.int16)
    assert np.array_equal(b.view(np.int16), want.numpy())


def test_stack():
    a, b = make_quant(1, "i4", 16, 256), make_quant(2, "i4", 32, 256)
    s = Quant.stack([a, b])
    assert s.rows == 48 and np.array_equal(s.q[16:], b.q) and np.array_equal(s.scales[:32], a.scales)
    with pytest.raises(ValueError):
        Quant.stack([a, make_quant(3, "i4", 16, 384)])


def test_dense_bf16_rejects():
    """Shape guards of the dense storage (rows of 16, columns of 128), and the int4/int8 unpacker refusing it."""
    from qwenny_amd._lib import QhError

    w = np.zeros((16, 100), np.uint16)
    with pytest.raises(QhError):
        packed_sizes(Wt.BF16, 16, 100)
    with pytest.raises(QhError):
        pack_dense_bf16(w, np.arange(16))
    with pytest.raises(QhError):
        pack_dense_bf16(np.zeros((24, 128), np.uint16), np.arange(24))  # 24 rows: not whole tiles
    codes = pack_dense_bf16(np.zeros((16, 128), np.uint16), np.arange(16))
    with pytest.raises(QhError):
        unpack_rows(Wt.BF16, 16, 128, codes, np.zeros(0, np.uint8))
    q = make_quant(5, "i4", 16, 128)
    with pytest.raises(QhError):
        pack_quant(q, np.arange(16), Wt.BF16)
