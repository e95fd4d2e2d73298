"""The matrix-product runtime: Python mirror of the reference's `Wt`, `Mat`, `Epi`, `Gemm` (src/cuda/core.rs:52-681)
over the C ABI of libqwenny_hip (include/qwenny_hip.h).

Same names, argument meanings and error behaviour as the reference: `Mat.stack` / `Mat.marlin` / `Mat.int8` /
`Mat.new` / `Mat.marlin_rows` build device matrices (shape guards raise), `Gemm.run` / `Gemm.run_split` launch a
product on a stream and return the split-K factor, `Gemm.put_block` rewrites one 16-row block. Device buffers (x, y,
keys, out_rows) are anything with `data_ptr()` (torch tensors) or raw device addresses.
"""

import ctypes
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from ._lib import MatDesc, QuantC, check, lib

P = ctypes.c_void_p


# Token counts the decode (skinny) kernel takes at most (csrc/kernels.h SKINNY_MAX_M; from 33 tokens the plain and
# SwiGLU products of int4 and grouped int8 matrices of 2^26 weights or more go to the prefill kernel instead:
# Mat.kernel says which kernel a product runs on). The skinny kernel's products are exact (every weight bf16 (128 + q)
# times x summed in f32, the scale after) and plain ones return split-K partials; the prefill kernel rounds each
# dequantized weight to bf16 once, and its plain products return 1-16 partials (K slices) up to 512 tokens, one above.
SKINNY_MAX_M = 48


class Wt(IntEnum):
    """How a matrix is stored (src/cuda/core.rs:65-79). I4 replaces Wt::Marlin, I4Z Wt::MarlinZ; the _S32 forms keep
    f32 scales (scales bf16 does not hold exactly)."""

    I8 = 1
    I4 = 2
    I4Z = 3
    I4_S32 = 4
    I4Z_S32 = 5
    BF16 = 6  # dense 16-bit weights kept bf16 (Wt::F16, which rounds them to f16)

    @property
    def has_zeros(self):
        return self in (Wt.I4Z, Wt.I4Z_S32)

    def bits(self):
        return {Wt.I8: 8, Wt.BF16: 16}.get(self, 4)


class Epi(IntEnum):
    """Epilogue of a product (src/cuda/core.rs:52-58)."""

    Plain = 0
    Silu = 1
    Argmax = 2


QG = 128
MAX_TOK = 2048
MAX_OUT = 64


def _ptr(t):
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return int(t)


def _stream(s):
    if s is None:
        import torch

        return torch.cuda.current_stream().cuda_stream
    if hasattr(s, "cuda_stream"):
        return s.cuda_stream
    return int(s)


def _np_ptr(a):
    return a.ctypes.data_as(P) if a is not None else None


@dataclass
class Quant:
    """A quantized matrix [rows][cols], affine: w = q * scale + offset per group of a row (src/checkpoint.rs:21-31).
    q: uint32 [rows][cols * bits / 32]; scales, offsets: float32 [rows * cols / group]."""

    bits: int
    group: int
    rows: int
    cols: int
    q: np.ndarray
    scales: np.ndarray
    offsets: np.ndarray

    def __post_init__(self):
        self.q = np.ascontiguousarray(self.q, np.uint32).reshape(self.rows, -1)
        self.scales = np.ascontiguousarray(self.scales, np.float32).reshape(-1)
        self.offsets = np.ascontiguousarray(self.offsets, np.float32).reshape(-1)
        if self.q.shape[1] * 32 != self.cols * self.bits or self.scales.size != self.rows * (self.cols // self.group):
            raise ValueError(f"quant {self.rows} x {self.cols}: {self.q.shape} words, {self.scales.size} scales")

    def c(self):
        return QuantC(self.bits, self.group, self.rows, self.cols, self.q.ctypes.data, self.scales.ctypes.data,
                      self.offsets.ctypes.data)

    def row_into(self, r):
        """Row r dequantized to f32 (src/checkpoint.rs:39-47)."""
        out = np.empty(self.cols, np.float32)
        check(lib().qh_quant_row_into(ctypes.byref(self.c()), r, _np_ptr(out)))
        return out

    def to_bf16(self):
        """All rows dequantized, as bf16 bits rounded to nearest even (src/checkpoint.rs:50-68), threaded over rows."""
        out = np.empty((self.rows, self.cols), np.uint16)
        check(lib().qh_quant_to_bf16(ctypes.byref(self.c()), _np_ptr(out)))
        return out

    def zero_points(self):
        """The integer zero point of each group if every offset is -z * scale (src/checkpoint.rs:72-82), else None."""
        z = np.empty(self.scales.size, np.uint8)
        return z if check(lib().qh_quant_zero_points(ctypes.byref(self.c()), _np_ptr(z))) == 1 else None

    @staticmethod
    def stack(parts):
        """Matrices with the same columns and quantization, stacked by rows (src/checkpoint.rs:85-99)."""
        parts = list(parts)
        if not parts:
            raise ValueError("nothing to stack")
        first = parts[0]
        for p in parts[1:]:
            if (p.bits, p.group, p.cols) != (first.bits, first.group, first.cols):
                raise ValueError("stacking differently quantized matrices")
        return Quant(first.bits, first.group, sum(p.rows for p in parts), first.cols,
                     np.concatenate([p.q for p in parts]), np.concatenate([p.scales for p in parts]),
                     np.concatenate([p.offsets for p in parts]))


def row_order(rows, silu):
    """Rows of a stacked matrix in the order they are packed (src/cuda/core.rs:108-114): `silu`: [w1; w3] (gate; up)
    interleaved so that each 16-row tile holds 8 rows of each."""
    out = np.empty(rows, np.uintp)
    check(lib().qh_row_order(rows, int(silu), _np_ptr(out)))
    return out.astype(np.int64)


class Gemm:
    """The product kernels on one device (src/cuda/core.rs:413-681 `Gemm`): `Gemm.load(device)`."""

    def __init__(self, ctx, device):
        self._ctx = ctx
        self.device = device

    @classmethod
    def load(cls, device=0):
        ctx = P()
        check(lib().qh_open(device, ctypes.byref(ctx)))
        return cls(ctx, device)

    def close(self):
        if self._ctx:
            lib().qh_close(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run(self, stream, n, w, x, y, epi=Epi.Plain, out_rows=None, n_out=0, keys=None, ldx=0):
        """y = w . x for the step's `n` tokens (Argmax: its `n_out` logit rows `out_rows`, keeping the running argmax
        in `keys`); split-K partial products for decode-sized steps. Returns the split factor (src/cuda/core.rs:485)."""
        return self.run_split(stream, n, w, x, y, epi, False, out_rows, n_out, keys, ldx)

    def run_split(self, stream, n, w, x, y, epi, whole, out_rows=None, n_out=0, keys=None, ldx=0):
        """run; `whole`: a plain product without split K (src/cuda/core.rs:497-561)."""
        return check(lib().qh_gemm(self._ctx, _stream(stream), w._m, _ptr(x), ldx, n, _ptr(out_rows), n_out, _ptr(y),
                                   int(epi), _ptr(keys), int(whole)))

    def run_lora(self, stream, n, w, x, y, epi, lora, whole=False, ldx=0):
        """run / run_split with an unmerged LoRA adapter's delta fused into the epilogue: `lora` = (xa, split, m_cols,
        b_f16, rank, tab, tok_slot, slot_scale) as lora_add takes them (device tensors). Plain: the delta on split 0;
        Silu: added to gate and up before the activation. Returns the split."""
        from ._lib import LoraC

        xa, split, m_cols, b, rank, tab, tok_slot, slot_scale = lora
        lc = LoraC(_ptr(xa), split, m_cols, _ptr(b), rank, _ptr(tab), _ptr(tok_slot), _ptr(slot_scale))
        return check(lib().qh_gemm_lora(self._ctx, _stream(stream), w._m, _ptr(x), ldx, n, _ptr(y), int(epi),
                                        int(whole), ctypes.byref(lc)))

    def put_block(self, stream, m, q, zeros, block, rows):
        """Write stored rows `rows` (16) of `q` as the 16-row block `block` of a matrix from Mat.marlin_rows, counting
        it as valid (src/cuda/core.rs:619-657)."""
        rows = np.ascontiguousarray(rows, np.uintp)
        zeros = np.ascontiguousarray(zeros, np.uint8)
        if rows.size != 16:
            raise ValueError(f"{rows.size} rows for a 16-row block")
        check(lib().qh_put_block(self._ctx, _stream(stream), m._m, ctypes.byref(q.c()), _np_ptr(zeros), block,
                                 _np_ptr(rows)))

    def part_len(self, mats, max_tok=MAX_TOK):
        """Floats the plain products of `mats` write at most (src/cuda/core.rs:315-318)."""
        arr = (P * len(mats))(*[m._m for m in mats])
        return lib().qh_part_len(self._ctx, arr, len(mats), max_tok)


class Mat:
    """A weight matrix packed for the kernels in the gfx950 tile layout (src/cuda/core.rs:94-104 `Mat`)."""

    def __init__(self, gemm, handle):
        self._gemm = gemm
        self._m = handle
        self._free = lib().qh_mat_free  # bound now: at interpreter exit the module globals may already be gone

    def __del__(self):
        if getattr(self, "_m", None):
            self._free(self._m)
            self._m = None

    def desc(self):
        d = MatDesc()
        check(lib().qh_mat_describe(self._m, ctypes.byref(d)))
        return d

    @property
    def wt(self):
        return Wt(self.desc().wt)

    @property
    def per_channel(self):
        """int8 with one scale per row: prefill products in exact integers, the row's scale after the sum."""
        return bool(self.desc().per_channel)

    @property
    def rows(self):
        return self.desc().rows

    @property
    def tiles(self):
        return self.rows // 16

    @property
    def cols(self):
        return self.desc().cols

    @property
    def valid(self):
        return self.desc().valid

    def split(self, n):
        """Split-K factor of a plain product of n tokens (src/cuda/core.rs Mat::split)."""
        return check(lib().qh_mat_split(self._gemm._ctx, self._m, n))

    def kernel(self, n, epi=None, whole=False):
        """"skinny" or "prefill": the kernel a product of n tokens (n_out logit rows for the argmax) with epilogue
        `epi` (Plain by default) runs on this matrix. The skinny kernel's products are exact products of the
        dequantized weights; the prefill kernel rounds each weight to bf16 once."""
        e = Epi.Plain if epi is None else epi
        k = check(lib().qh_mat_kernel(self._gemm._ctx, self._m, n, int(e), int(bool(whole))))
        return "skinny" if k == 1 else "prefill"

    def download(self):
        """The packed buffers (codes, scales, zeros) back on the host."""
        d = self.desc()
        codes = np.empty(d.code_bytes, np.uint8)
        scales = np.empty(d.scale_bytes, np.uint8)
        zeros = np.empty(d.zero_bytes, np.uint8) if d.zero_bytes else None
        check(lib().qh_mat_download(self._m, _np_ptr(codes), _np_ptr(scales), _np_ptr(zeros)))
        return codes, scales, zeros

    @classmethod
    def marlin(cls, gemm, q, silu=False):
        """A stored int4 matrix (integer zero points, groups of a multiple of 128, rows of 16, columns of 128) in the
        tile layout, or None if it does not fit (src/cuda/core.rs:155-164)."""
        if q.bits != 4:
            return None
        return cls._quant(gemm, q, silu)

    @classmethod
    def int8(cls, gemm, q, silu=False):
        """A stored symmetric int8 matrix (zero point 128) as it is, or None (src/cuda/core.rs:166-191)."""
        if q.bits != 8:
            return None
        return cls._quant(gemm, q, silu)

    @classmethod
    def _quant(cls, gemm, q, silu):
        h = P()
        rc = lib().qh_mat_quant(gemm._ctx, ctypes.byref(q.c()), int(silu), ctypes.byref(h))
        if rc == -4:  # QH_ENOTFIT
            return None
        check(rc)
        return cls(gemm, h)

    @classmethod
    def marlin_rows(cls, gemm, q, zeros, rows, cap):
        """Rows `rows` (whole tiles) of a stored int4 matrix in a matrix of `cap` rows: the rest are room for later
        rows (Gemm.put_block), not valid (src/cuda/core.rs:136-153)."""
        rows = np.ascontiguousarray(rows, np.uintp)
        zeros = np.ascontiguousarray(zeros, np.uint8)
        h = P()
        check(lib().qh_mat_quant_rows(gemm._ctx, ctypes.byref(q.c()), _np_ptr(zeros), _np_ptr(rows), rows.size, cap,
                                      ctypes.byref(h)))
        return cls(gemm, h)

    @classmethod
    def new(cls, gemm, w_bf16, cols, silu=False, int8=True):
        """Pack dense bf16 [rows][cols] (src/cuda/core.rs:126-135): requantized to int8 (Wt.I8), or with int8 False
        kept 16-bit (Wt.BF16; the reference's Wt::F16 rounds to f16, here the bf16 values stay as they are)."""
        w = np.ascontiguousarray(w_bf16, np.uint16).reshape(-1, cols)
        h = P()
        fn = lib().qh_mat_dense_int8 if int8 else lib().qh_mat_dense
        check(fn(gemm._ctx, _np_ptr(w), w.shape[0], cols, int(silu), ctypes.byref(h)))
        return cls(gemm, h)

    @classmethod
    def from_checkpoint(cls, gemm, ck, names, silu=False, int8=True):
        """Matrices `names` (`.weight`) of a checkpoint with the same column count, stacked by rows
        (src/cuda/core.rs:193-219 Mat::stack): stored quantized ones as Mat.stack takes them; else dense, requantized
        to int8 when `int8` unless the checkpoint is pre-quantized (its 16-bit matrices stay 16-bit)."""
        bases = [n[:-len(".weight")] for n in names if n.endswith(".weight")]
        if len(bases) == len(names) and all(ck.is_quant(b) for b in bases):
            return cls.stack(gemm, [ck.quant_matrix(b) for b in bases], silu, int8)
        parts = [ck.bf16(n) for n in names]
        cols = parts[0][1][1]
        if any(shape[1] != cols for _, shape in parts):
            raise ValueError(f"{names[0]}: stacking matrices of different column counts")
        dense = np.concatenate([w.reshape(-1, cols) for w, _ in parts])
        return cls.new(gemm, dense, cols, silu, int8 and not ck.prequantized())

    @classmethod
    def stack(cls, gemm, parts, silu=False, int8=True):
        """Matrices with the same column count stacked by rows (src/cuda/core.rs:193-219): stored int4 in the tile
        layout (an error where it does not fit), stored int8 as it is; else dense bf16 requantized to int8.
        `parts`: Quant objects, or (bf16 array, cols) pairs for dense matrices."""
        if all(isinstance(p, Quant) for p in parts):
            q = Quant.stack(parts)
            if q.bits == 4:
                m = cls.marlin(gemm, q, silu)
                if m is None:
                    raise ValueError(f"int4 of {q.rows} x {q.cols} in groups of {q.group}: the tile layout needs rows "
                                     "a multiple of 16, columns of 128 and groups of a multiple of 128 with integer "
                                     "zero points")
                return m
            m = cls.int8(gemm, q, silu)
            if m is not None:
                return m
            dense = q.to_bf16()
            return cls.new(gemm, dense, q.cols, silu, int8)
        cols = parts[0][1]
        dense = np.concatenate([np.asarray(w, np.uint16).reshape(-1, cols) for w, _ in parts])
        return cls.new(gemm, dense, cols, silu, int8)


def packed_sizes(wt, rows, cols):
    """(code, scale, zero) bytes of the tile layout."""
    c, s, z = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    check(lib().qh_packed_sizes(int(wt), rows, cols, ctypes.byref(c), ctypes.byref(s), ctypes.byref(z)))
    return c.value, s.value, z.value


def pack_quant(q, order, wt, zeros=None):
    """The load-time repacker on the host: rows `order` of `q` into the tile layout -> (codes, scales, zeros) bytes."""
    order = np.ascontiguousarray(order, np.uintp)
    cb, sb, zb = packed_sizes(wt, order.size, q.cols)
    codes, scales = np.empty(cb, np.uint8), np.empty(sb, np.uint8)
    zs = np.empty(zb, np.uint8) if zb else None
    zin = None if zeros is None else np.ascontiguousarray(zeros, np.uint8)
    check(lib().qh_pack_quant(ctypes.byref(q.c()), _np_ptr(zin), _np_ptr(order), order.size, int(wt), _np_ptr(codes),
                              _np_ptr(scales), _np_ptr(zs)))
    return codes, scales, zs


def unpack_rows(wt, rows, cols, codes, scales, zeros=None):
    """The repacker's inverse: (values u8 [rows][cols], scales f32 [rows][cols/128], zeros u8 [rows][cols/128])."""
    vals = np.empty((rows, cols), np.uint8)
    sc = np.empty((rows, cols // QG), np.float32)
    z = np.empty((rows, cols // QG), np.uint8)
    for p in range(rows):
        check(lib().qh_unpack_row(int(wt), rows, cols, _np_ptr(codes), _np_ptr(scales), _np_ptr(zeros), p,
                                  _np_ptr(vals[p]), _np_ptr(sc[p]), _np_ptr(z[p])))
    return vals, sc, z


def dequant(stream, q, scales, zeros, rows, words, cols, group, bits, r0, n, out, out_f32=False):
    """The trainer's dequant (kernels/qwen_train.cu:84-103): rows [r0, r0 + n) of a quantized matrix in the
    checkpoint's layout, all device buffers (q u32 [rows][words], scales f32 and zeros u8 per (row, group)), into
    dense rows `out` [n][cols], bf16 or f32, on `stream`."""
    check(lib().qh_dequant(_stream(stream), _ptr(q), _ptr(scales), _ptr(zeros), rows, words, cols, group, bits, r0,
                           n, _ptr(out), int(out_f32)))


def diag_read(stream, buf, tiles, groups, pattern, sink):
    """The measurement aid qh_diag_read: a read-only pass over tiles x groups 1 KiB blocks of `buf` with the decode
    kernel's loads (pattern 0 contiguous, 1 the one-token product's tile walk), storing nothing; `sink` a device u32."""
    check(lib().qh_diag_read(_stream(stream), _ptr(buf), tiles, groups, int(pattern), _ptr(sink)))


def sum_parts(stream, x, splits, n, ld, y):
    """y [n][ld] = the sum of a plain product's `splits` partials x [splits][n][ld] (kernels/qwen.cu:141-143)."""
    check(lib().qh_sum_parts(_stream(stream), _ptr(x), splits, n, ld, _ptr(y)))


def add_rmsnorm(stream, h, x, splits, n, hidden, w_next, y, eps=1e-6):
    """The residual step after a plain product (kernels/qwen.cu:57-80): h [n][hidden] += the sum of the partials x,
    then y [n][hidden] bf16 = w_next * h / rms(h)."""
    check(lib().qh_add_rmsnorm(_stream(stream), _ptr(h), _ptr(x), splits, n, hidden, _ptr(w_next), _ptr(y), eps))


def lora_add(stream, xa, split, m_cols, b_f16, rank, rows, tab, tok_slot, slot_scale, n, y, ldy=0):
    """An unmerged LoRA adapter's delta on a plain product (kernels/lora.cuh:52-76, src/cuda/qwen/lora.rs:178-180):
    y [n][ldy] (split 0) row o += s_t * B[o] . xa[t][off(o) ..] for the tokens of adapter slots; all device buffers."""
    check(lib().qh_lora_add(_stream(stream), _ptr(xa), split, m_cols, _ptr(b_f16), rank, rows, _ptr(tab),
                            _ptr(tok_slot), _ptr(slot_scale), n, _ptr(y), ldy or rows))


def lora_silu(stream, xa, split, m_cols, b_f16, rank, rows, tab, tok_slot, slot_scale, n, y, mid, ldy=0):
    """SwiGLU of a plain [gate; up] product with the adapter's delta added first (kernels/lora.cuh:78-113,
    src/cuda/qwen/lora.rs:184-187): mid [n][rows / 2] bf16; all device buffers."""
    check(lib().qh_lora_silu(_stream(stream), _ptr(xa), split, m_cols, _ptr(b_f16), rank, rows, _ptr(tab),
                             _ptr(tok_slot), _ptr(slot_scale), n, _ptr(y), ldy or rows, _ptr(mid)))


def pack_dense_bf16(w_bf16, order):
    """Dense bf16 rows `order` in the QH_WT_BF16 tile layout (src/cuda/core.rs:370-381, kept bf16) -> codes bytes."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    order = np.ascontiguousarray(order, np.uintp)
    cb, _, _ = packed_sizes(Wt.BF16, order.size, w.shape[1])
    codes = np.empty(cb, np.uint8)
    check(lib().qh_pack_dense_bf16(_np_ptr(w), w.shape[0], w.shape[1], _np_ptr(order), order.size, _np_ptr(codes)))
    return codes


def unpack_rows_bf16(rows, cols, codes):
    """The QH_WT_BF16 packer's inverse: bf16 bits [rows][cols] in packed row order."""
    out = np.empty((rows, cols), np.uint16)
    for p in range(rows):
        check(lib().qh_unpack_row_bf16(rows, cols, _np_ptr(codes), p, _np_ptr(out[p])))
    return out


def pack_dense_int8(w_bf16, order):
    """Requantize dense bf16 rows `order` to int8 in the tile layout (src/cuda/core.rs:356-369) -> (codes, scales)."""
    w = np.ascontiguousarray(w_bf16, np.uint16)
    order = np.ascontiguousarray(order, np.uintp)
    cb, sb, _ = packed_sizes(Wt.I8, order.size, w.shape[1])
    codes, scales = np.empty(cb, np.uint8), np.empty(sb, np.uint8)
    check(lib().qh_pack_dense_int8(_np_ptr(w), w.shape[0], w.shape[1], _np_ptr(order), order.size, _np_ptr(codes),
                                   _np_ptr(scales)))
    return codes, scales


class Graph:
    """A captured sequence of launches (the capture and replay inside src/cuda/core.rs:1151-1192 `Graphs::run`):

        g = Graph.capture(stream, lambda: gemm.run(stream, ...))
        g.launch(stream)

    `stream`: a torch stream (not the null stream) or a hipStream_t as an int."""

    def __init__(self, handle):
        self._g = handle

    @classmethod
    def capture(cls, stream, fn):
        s = _stream(stream)
        check(lib().qh_graph_begin(s))
        h = P()
        try:
            fn()
        except BaseException:
            if lib().qh_graph_end(s, ctypes.byref(h)) == 0:  # the capture ends either way
                lib().qh_graph_free(h)
            raise
        check(lib().qh_graph_end(s, ctypes.byref(h)))
        return cls(h)

    def launch(self, stream):
        check(lib().qh_graph_launch(self._g, _stream(stream)))

    def close(self):
        if self._g:
            lib().qh_graph_free(self._g)
            self._g = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
