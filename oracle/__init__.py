"""CPU oracle of qwenny's quantized-weight products — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only as the checker
(or the timed CPU baseline), never as the thing shipped: the product (qwenny_amd) never imports it.

ctypes bindings of oracle.c (the C restatement, built by oracle/Makefile) plus numpy restatements of the small
epilogue pieces. Every function cites the reference file:line it follows (paths relative to the reference repository).

Pinning: every function is checked in tests/test_oracle.py against hand-built known answers, closed forms, library
routines (numpy f64 matmul, torch's bf16 rounding and SiLU) or the reference's own known-answer generator
(src/mlx/metal.rs:375-384). Nothing here is "parity unpinned".
"""

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
        P, S, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
        _lib.or_packed_matrix.argtypes = [P, S, S, S, I, I, P, P, S, S, P, P, P, P, P]
        _lib.or_packed_matrix.restype = I
        _lib.or_row_into.argtypes = [I, S, S, P, P, P, S, P]
        _lib.or_zero_points.argtypes = [I, S, P, P, P]
        _lib.or_zero_points.restype = I
        _lib.or_row_order.argtypes = [S, I, P]
        _lib.or_requant_int8.argtypes = [P, S, S, P, P]
        _lib.or_gemm_f64.argtypes = [I, S, S, S, P, P, P, P, S, P, I]
        _lib.or_gemm_f32.argtypes = [I, S, S, S, P, P, P, P, S, P, I]
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def packed_matrix(weight_packed, weight_scale, bits, group, cols=0, zero_point=None):
    """Checkpoint::packed_matrix (src/checkpoint.rs:408-453) -> (bits, group, cols, scales f32, offsets f32)."""
    wp = np.ascontiguousarray(weight_packed, dtype=np.uint32)
    rows, words = wp.shape
    sc = np.ascontiguousarray(weight_scale, dtype=np.float32).reshape(-1)
    zp = None if zero_point is None else np.ascontiguousarray(zero_point, dtype=np.uint32)
    out_s = np.empty(sc.size, np.float32)
    out_o = np.empty(sc.size, np.float32)
    b, g, c = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_size_t()
    rc = lib().or_packed_matrix(_p(wp), rows, words, cols, bits, group, _p(sc), _p(zp),
                                0 if zp is None else zp.shape[0], 0 if zp is None else zp.shape[1],
                                _p(out_s), _p(out_o), ctypes.byref(b), ctypes.byref(g), ctypes.byref(c))
    if rc != 0:
        raise ValueError("packed matrix does not fit compressed-tensors' packing")
    return b.value, g.value, c.value, out_s, out_o


def row_into(bits, group, cols, q, scales, offsets, r):
    """Quant::row_into (src/checkpoint.rs:39-47): row r as f32."""
    out = np.empty(cols, np.float32)
    lib().or_row_into(bits, group, cols, _p(np.ascontiguousarray(q, np.uint32)),
                      _p(np.ascontiguousarray(scales, np.float32)), _p(np.ascontiguousarray(offsets, np.float32)),
                      r, _p(out))
    return out


def zero_points(bits, scales, offsets):
    """Quant::zero_points (src/checkpoint.rs:72-82): uint8 array or None."""
    s = np.ascontiguousarray(scales, np.float32).reshape(-1)
    o = np.ascontiguousarray(offsets, np.float32).reshape(-1)
    z = np.empty(s.size, np.uint8)
    return z if lib().or_zero_points(bits, s.size, _p(s), _p(o), _p(z)) else None


def row_order(rows, silu):
    """row_order (src/cuda/core.rs:108-114)."""
    out = np.empty(rows, np.uintp)
    lib().or_row_order(rows, int(silu), _p(out))
    return out.astype(np.int64)


def requant_int8(w_bf16):
    """Mat::new int8 branch (src/cuda/core.rs:356-369): (stored values u8 [rows][cols], scales f32 [rows][cols/128])."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    rows, cols = w.shape
    vals = np.empty((rows, cols), np.uint8)
    sc = np.empty((rows, cols // 128), np.float32)
    lib().or_requant_int8(_p(w), rows, cols, _p(vals), _p(sc))
    return vals, sc


def gemm_f64(bits, group, q, scales, offsets, x_bf16, threads=None):
    """y[t][r] = sum_c x[t][c] (q - z) s in f64 (src/checkpoint.rs:39-47 semantics); x bf16 bits [m][cols]."""
    q = np.ascontiguousarray(q, np.uint32)
    rows, words = q.shape
    cols = words * 32 // bits
    x = np.ascontiguousarray(x_bf16, np.uint16).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float64)
    lib().or_gemm_f64(bits, group, rows, cols, _p(q), _p(np.ascontiguousarray(scales, np.float32)),
                      _p(np.ascontiguousarray(offsets, np.float32)), _p(x), x.shape[0], _p(y),
                      threads or os.cpu_count() or 1)
    return y


def gemm_f32(bits, group, q, scales, offsets, x_bf16, threads=1):
    """The reference's CPU form: Quant::row_into to f32, then a plain f32 dot (the benchmark's CPU baseline)."""
    q = np.ascontiguousarray(q, np.uint32)
    rows, words = q.shape
    cols = words * 32 // bits
    x = np.ascontiguousarray(x_bf16, np.uint16).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), np.float32)
    lib().or_gemm_f32(bits, group, rows, cols, _p(q), _p(np.ascontiguousarray(scales, np.float32)),
                      _p(np.ascontiguousarray(offsets, np.float32)), _p(x), x.shape[0], _p(y), threads)
    return y


def dense_f64(w_bf16, x_bf16, f16_weights=False):
    """The dense 16-bit product y[t][r] = sum_c x[t][c] w[r][c] in f64 (src/cuda/core.rs:370-381 packs the weights,
    kernels/gemm.cuh:120-212 multiplies them); w, x bf16 bits. `f16_weights`: the reference's storage, which rounds
    each weight to f16 (half::f16::from_f32, nearest even) before the product."""
    w = np.asarray(w_bf16, np.uint16).astype(np.uint32) << 16
    w = w.view(np.float32)
    if f16_weights:
        with np.errstate(over="ignore"):  # beyond 65504: infinity, as the reference's f16 storage
            w = w.astype(np.float16).astype(np.float32)
    x = (np.asarray(x_bf16, np.uint16).astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float64) @ w.astype(np.float64).T


def dequant_rows(bits, group, q, scales, zeros, r0, n, out_f32=False):
    """The trainer's dequant (kernels/qwen_train.cu:84-103): rows [r0, r0 + n) of q (u32 [rows][words], value c in
    word c * bits / 32 from the low bits) as ((float) q - zero) * scale in f32 per (row, group), then bf16 bits
    (nearest even, the bf16 build's to_act) or f32."""
    per = 32 // bits
    q = np.asarray(q, np.uint32)[r0:r0 + n]
    cols = q.shape[1] * per
    c = np.arange(cols)
    vals = ((q[:, c // per] >> ((c % per) * bits).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.float32)
    g = cols // group
    s = np.asarray(scales, np.float32).reshape(-1, g)[r0:r0 + n][:, c // group]
    z = np.asarray(zeros, np.uint8).reshape(-1, g)[r0:r0 + n][:, c // group].astype(np.float32)
    w = (vals - z) * s  # f32: the difference is exact, the product rounds once
    if out_f32:
        return w
    u = w.view(np.uint32).astype(np.uint64)  # round to nearest even (no NaN arises from finite inputs)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def sum_parts(x, splits):
    """kernels/qwen.cu:141-143 (part_sum, kernels/common.cuh:66-70): the partials x [splits][n][ld] summed in f32 from
    0, split 0 first."""
    x = np.asarray(x, np.float32)
    v = np.zeros(x.shape[1:], np.float32)
    for s in range(splits):
        v = v + x[s]
    return v


def add_rmsnorm(h, x, splits, w_next, eps):
    """kernels/qwen.cu:57-80: h + x[0] + x[1] + .. in f32 (that order), then w * h / sqrt(mean(h^2) + eps) in f64;
    returns (new h f32, y f64)."""
    v = np.asarray(h, np.float32).copy()
    x = np.asarray(x, np.float32)
    for s in range(splits):
        v = v + x[s]
    d = v.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(d * d, axis=-1, keepdims=True) + eps)
    return v, np.asarray(w_next, np.float64) * (d * r)


def _lora_delta(xa, split, b_f16, rank, tab, tok_slot, slot_scale, n, rows_of):
    """kernels/lora.cuh:13-46: per token the slot's scale s_t (0: no delta), xa summed over the splits (f32, split 0
    first), and for output row o of module mod(o) (tab[0..3] end rows) with first column off = tab[4 + mod] >= 0 the
    delta s_t * B[o] . xa[t][off .. off + rank) (f64 here). Returns (delta f64 [n][len(rows_of)], scales f32 [n])."""
    xa = np.asarray(xa, np.float32)
    m = xa.shape[-1]
    xs = np.zeros((n, m), np.float32)
    for s in range(split):
        xs = xs + xa[s, :n]
    sc = np.asarray(slot_scale, np.float32)[np.asarray(tok_slot)[:n]]
    b = np.asarray(b_f16, np.uint16).view(np.float16).astype(np.float64).reshape(-1, rank)
    delta = np.zeros((n, len(rows_of)), np.float64)
    for i, o in enumerate(rows_of):
        mod = int(o >= tab[0]) + int(o >= tab[1]) + int(o >= tab[2])
        off = tab[4 + mod]
        if off < 0:
            continue
        delta[:, i] = xs[:, off:off + rank].astype(np.float64) @ b[o]
    return delta * sc[:, None].astype(np.float64), sc


def lora_add(y, xa, split, b_f16, rank, tab, tok_slot, slot_scale, n):
    """kernels/lora.cuh:52-76 (lora_add): y [n][rows] (a plain product's split 0) + s_t B (A x) for the tokens of
    adapter slots; f64."""
    y = np.asarray(y, np.float64)
    delta, sc = _lora_delta(xa, split, b_f16, rank, tab, tok_slot, slot_scale, n, range(y.shape[1]))
    return np.where(sc[:, None] != 0, y[:n] + delta, y[:n])


def lora_silu(y, xa, split, b_f16, rank, tab, tok_slot, slot_scale, n):
    """kernels/lora.cuh:78-113 (lora_silu): y [n][rows] a plain [gate; up] product packed in the SwiGLU row order
    (16-row tile p: gate rows 8p .. 8p + 7, then their up rows); mid [n][rows / 2] = silu(gate + dg) * (up + du) in
    f64, output j from packed rows 16 (j / 8) + j % 8 and + 8. Only tab[4] (gate) and tab[5] (up) are read."""
    y = np.asarray(y, np.float64)[:n]
    rows = y.shape[1]
    j = np.arange(rows // 2)
    og = 16 * (j // 8) + j % 8
    ou = og + 8
    t8 = [2**31 - 1] * 4 + [tab[4], -1, -1, -1]
    dg, sc = _lora_delta(xa, split, b_f16, rank, t8, tok_slot, slot_scale, n, og)
    t8 = [2**31 - 1] * 4 + [tab[5], -1, -1, -1]
    du, _ = _lora_delta(xa, split, b_f16, rank, t8, tok_slot, slot_scale, n, ou)
    g, u = y[:, og] + dg, y[:, ou] + du
    return g / (1.0 + np.exp(-g)) * u


# ---- epilogues (numpy restatements) ---------------------------------------------------------------------------


def silu_glu(y_f64, order):
    """SwiGLU epilogue (kernels/gemm.cuh:83-91, kernels/marlin.cuh:490-492 with row_order src/cuda/core.rs:108-114):
    y [m][rows] in ORIGINAL row order ([gate; up]) -> silu(gate) * up [m][rows/2]."""
    del order  # the oracle works in original row order: gate rows 0..rows/2, up rows rows/2..rows
    half = y_f64.shape[1] // 2
    g, u = y_f64[:, :half], y_f64[:, half:]
    return g / (1.0 + np.exp(-g)) * u


def ordered(v):
    """ordered() (kernels/common.cuh:60-63): order-preserving float -> u32."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def argmax_keys(logits_f32, valid):
    """The argmax key per logit row (kernels/gemm.cuh:72-74, kernels/marlin.cuh:499-517):
    max over rows o < valid of (ordered(v) << 32) | (0xffffffff - o): the largest value, lowest index on ties."""
    lg = np.asarray(logits_f32, np.float32)[:, :valid]
    idx = np.arange(valid, dtype=np.uint64)
    keys = (ordered(lg) << np.uint64(32)) | (np.uint64(0xFFFFFFFF) - idx)[None, :]
    return keys.max(axis=1)
