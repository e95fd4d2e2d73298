"""A checkpoint's quantized matrices as stored: compressed-tensors pack-quantized safetensors, read into `Quant`
(src/checkpoint.rs:21-99, :129-180, :196-453 — only the pieces the quantized products need).

Safetensors files are read by parsing their JSON header and memory-mapping the data (numpy has no bf16 dtype, so
16-bit floats are converted explicitly); nothing in a file is executed.
"""

import json
import os
import struct

import numpy as np

from ._lib import QuantC, check, lib
from .core import Quant
from .synth import bf16_to_f32, f32_to_bf16


def packed_scheme(qc):
    """compressed-tensors' quantization_config -> (bits, group) of its weight scheme (src/checkpoint.rs:129-180):
    pack-quantized, int, 4 or 8 bits, grouped or per channel (group 0), no activation quantization, no g_idx."""
    if qc.get("format") != "pack-quantized":
        raise ValueError(f"compressed-tensors format {qc.get('format')!r}: pack-quantized only")
    groups = qc.get("config_groups")
    if not isinstance(groups, dict):
        raise ValueError("config_groups")
    schemes = []
    for g in groups.values():
        if g.get("input_activations") is not None:
            raise ValueError("activation quantization is not supported: weights only")
        w = g.get("weights") or {}
        if w.get("type") != "int":
            raise ValueError(f"compressed-tensors weights of type {w.get('type')!r}: int only")
        bits = w.get("num_bits")
        if bits not in (4, 8):
            raise ValueError(f"{bits}-bit weights: 4 or 8")
        strategy = w.get("strategy")
        if strategy == "group":
            group = w.get("group_size")
            if not isinstance(group, int):
                raise ValueError("group_size")
        elif strategy == "channel":
            group = 0
        else:
            raise ValueError(f"compressed-tensors strategy {strategy!r}: group or channel")
        act = w.get("actorder")
        if not (act is None or act in ("static", "weight") or act is False):
            raise ValueError(f"actorder {act!r}: activation-ordered groups (g_idx) are not supported")
        schemes.append((bits, group))
    if not schemes:
        raise ValueError("no compressed-tensors config groups")
    bits, group = schemes[0]
    if not (all(s[1] == group for s in schemes) and (len(schemes) == 1 or group > 0)):
        raise ValueError(f"compressed-tensors config groups of different group sizes: {schemes}")
    return bits, group


def _floats(arr, dtype):
    """float_format (src/checkpoint.rs:186-193): bf16 / f16 / f32 values as f32."""
    if dtype == "BF16":
        return bf16_to_f32(arr.view(np.uint16))
    if dtype == "F16":
        return arr.view(np.float16).astype(np.float32)
    if dtype == "F32":
        return arr.view(np.float32).astype(np.float32)
    raise ValueError(f"{dtype} is not a float tensor")


def quant_from_packed(weight_packed, weight_scale, bits, group, zero_point=None, weight_shape=None):
    """Checkpoint::packed_matrix (src/checkpoint.rs:408-453) on in-memory tensors: weight_packed int32 [rows][words],
    weight_scale as f32 (any shape of rows * groups values), zero_point int32 words or None, weight_shape [rows, cols]
    or None -> Quant."""
    wp = np.ascontiguousarray(weight_packed).view(np.uint32).reshape(weight_packed.shape[0], -1)
    rows, words = wp.shape
    sc = np.ascontiguousarray(weight_scale, np.float32).reshape(-1)
    cols = 0
    if weight_shape is not None:
        ws = [int(v) for v in np.asarray(weight_shape).reshape(-1)]
        if len(ws) != 2 or ws[0] != rows:
            raise ValueError(f"weight_shape {ws} for {rows} packed rows")
        cols = ws[1]
    zp = None if zero_point is None else np.ascontiguousarray(zero_point).view(np.uint32).reshape(zero_point.shape[0], -1)
    scales = np.empty(sc.size, np.float32)
    offsets = np.empty(sc.size, np.float32)
    out = QuantC()
    check(lib().qh_quant_from_packed(wp.ctypes.data, rows, words, cols, bits, group, sc.ctypes.data,
                                     None if zp is None else zp.ctypes.data, 0 if zp is None else zp.shape[0],
                                     0 if zp is None else zp.shape[1], scales.ctypes.data, offsets.ctypes.data, out))
    if sc.size != out.rows * (out.cols // out.group):
        raise ValueError(f"weight_scale of {sc.size} values for {out.rows} rows of {out.cols // out.group} groups")
    return Quant(out.bits, out.group, out.rows, out.cols, wp, scales, offsets)


class SafeTensors:
    """One .safetensors file: header parsed, data memory-mapped read-only."""

    DTYPES = {"I32": np.int32, "U32": np.uint32, "I64": np.int64, "BF16": np.uint16, "F16": np.uint16,
              "F32": np.float32, "U8": np.uint8, "I8": np.int8}

    def __init__(self, path):
        with open(path, "rb") as f:
            (n,) = struct.unpack("<Q", f.read(8))
            self.meta = json.loads(f.read(n))
        self.meta.pop("__metadata__", None)
        self.data = np.memmap(path, dtype=np.uint8, mode="r", offset=8 + n)

    def names(self):
        return list(self.meta)

    def get(self, name):
        m = self.meta[name]
        lo, hi = m["data_offsets"]
        arr = np.frombuffer(self.data[lo:hi], dtype=self.DTYPES[m["dtype"]]).reshape(m["shape"])
        return m["dtype"], arr


def save_safetensors(path, tensors):
    """Write {name: (dtype, array)} as a .safetensors file (test fixtures and synthetic checkpoints)."""
    header, blobs, off = {}, [], 0
    for name, (dtype, arr) in tensors.items():
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    h += b" " * ((-len(h)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


class Checkpoint:
    """A compressed-tensors checkpoint directory (src/checkpoint.rs:196-264): config.json with quantization_config and
    one or more .safetensors files; tensor names without the `language_model.` prefix."""

    def __init__(self, path):
        with open(os.path.join(path, "config.json")) as f:
            config = json.load(f)
        qc = config.get("quantization_config") or (config.get("text_config") or {}).get("quantization_config")
        self.scheme = packed_scheme(qc) if qc else None
        files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
        self.files = [SafeTensors(os.path.join(path, f)) for f in files]
        self.index, self.prefix = {}, ""
        for i, st in enumerate(self.files):
            for n in st.names():
                self.index[n] = i
        if not any(n.startswith("model.") for n in self.index) and any(
                n.startswith("language_model.") for n in self.index):
            self.prefix = "language_model."

    def _raw(self, name):
        full = self.prefix + name if self.prefix and not name.startswith(self.prefix) else name
        if full not in self.index:
            return None
        return self.files[self.index[full]].get(full)

    def has(self, name):
        return self._raw(name) is not None

    def is_quant(self, base):
        """A matrix stored quantized (src/checkpoint.rs:284-297)."""
        return self.scheme is not None and self.has(base + ".weight_packed")

    def prequantized(self):
        return self.scheme is not None

    def bf16(self, name):
        """A 16-bit or f32 tensor as bf16 bits and its shape (src/checkpoint.rs Checkpoint::bf16): bf16 as stored,
        f16 and f32 rounded to nearest even."""
        raw = self._raw(name)
        if raw is None:
            raise KeyError(name)
        dt, arr = raw
        bits = arr.view(np.uint16) if dt == "BF16" else f32_to_bf16(_floats(arr, dt))
        return np.ascontiguousarray(bits).reshape(arr.shape), list(arr.shape)

    def quant_matrix(self, base):
        """The quantized matrix `{base}.weight` as stored (src/checkpoint.rs:370-375)."""
        if self.scheme is None:
            raise ValueError(f"{base} is stored quantized but config.json has no quantization")
        bits, group = self.scheme
        _, wp = self._raw(base + ".weight_packed")
        sdt, sc = self._raw(base + ".weight_scale")
        zp = self._raw(base + ".weight_zero_point")
        ws = self._raw(base + ".weight_shape")
        shape = ws[1] if ws is not None and ws[0] == "I64" else None
        return quant_from_packed(wp, _floats(sc, sdt), bits, group, None if zp is None else zp[1], shape)
