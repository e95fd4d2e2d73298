"""Seeded synthetic inputs of the benchmark configurations, in the checkpoint's own form (compressed-tensors
pack-quantized tensors), plus bf16 helpers.

Every tensor comes from its own numpy MT19937 stream seeded from (config seed, tensor name), so any one tensor can be
regenerated alone.
"""

import zlib

import numpy as np


def f32_to_bf16(a):
    """float32 -> bf16 bits (uint16), round to nearest even."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def rng(seed, name):
    return np.random.Generator(np.random.MT19937(seed * 1_000_003 + zlib.crc32(name.encode())))


def int4_packed(seed, name, n, k):
    """weight_packed int32 [n][k / 8]: codes uniform in 0..15 (signed -8..7 stored + 8), 8 per word along k, value c
    at bits 4 (c % 8). Uniform 32-bit words give exactly that."""
    return rng(seed, name + ".weight_packed").integers(0, 1 << 32, size=(n, k // 8), dtype=np.uint32)


def int8_packed(seed, name, n, k):
    """weight_packed int32 [n][k / 4]: int8 uniform in -127..127 stored + 128, 4 per word along k."""
    b = rng(seed, name + ".weight_packed").integers(1, 256, size=(n, k), dtype=np.uint8)
    return b.view(np.uint32).reshape(n, k // 4).copy()


def scales_bf16(seed, name, shape, lo, hi):
    """bf16 scales U(lo, hi) as bf16 bits."""
    return f32_to_bf16(rng(seed, name + ".weight_scale").uniform(lo, hi, size=shape).astype(np.float32))


def zero_points_packed(seed, name, n, groups):
    """weight_zero_point int32 [ceil(n / 8)][groups]: zero points uniform in 0..15 packed 8 per word along the rows
    (compressed-tensors' packed_dim 0); returns (packed, unpacked u8 [n][groups])."""
    z = rng(seed, name + ".weight_zero_point").integers(0, 16, size=(n, groups), dtype=np.uint32)
    pad = (-n) % 8
    zp = np.concatenate([z, np.zeros((pad, groups), np.uint32)]).reshape(-1, 8, groups)
    packed = np.zeros((zp.shape[0], groups), np.uint32)
    for i in range(8):
        packed |= zp[:, i, :] << np.uint32(4 * i)
    return packed, z.astype(np.uint8)


def activations(seed, name, m, k, outliers=0.0):
    """x bf16 [m][k] ~ N(0, 1); with `outliers`, that fraction of columns multiplied by 20."""
    r = rng(seed, name + ".x")
    x = r.standard_normal((m, k), dtype=np.float32)
    if outliers:
        cols = r.choice(k, size=max(1, int(round(k * outliers))), replace=False)
        x[:, cols] *= 20.0
    return f32_to_bf16(x)


def int4_quant(seed, name, n, k, zp=False, group=128):
    """A synthetic int4 matrix as the checkpoint stores it -> dict of compressed-tensors tensors."""
    t = {
        "weight_packed": int4_packed(seed, name, n, k),
        "weight_scale": scales_bf16(seed, name, (n, k // group), 0.002, 0.02),
        "weight_shape": np.array([n, k], np.int64),
    }
    if zp:
        t["weight_zero_point"], _ = zero_points_packed(seed, name, n, k // group)
    return t


def int8_quant(seed, name, n, k, group=0):
    """A synthetic int8 matrix -> compressed-tensors tensors: per channel (group 0, strategy "channel": one scale per
    row, U(0.001, 0.01)) or per group of `group` columns (strategy "group", scales U(0.001, 0.01) per row and group)."""
    return {
        "weight_packed": int8_packed(seed, name, n, k),
        "weight_scale": scales_bf16(seed, name, (n, k // group if group else 1), 0.001, 0.01),
        "weight_shape": np.array([n, k], np.int64),
    }
