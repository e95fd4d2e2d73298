"""Shared pieces of the tests: synthetic matrices in the checkpoint's form, the oracle's answer, the GPU product's
answer, and the parity bar."""

import numpy as np

import oracle
from qwenny_amd import synth
from qwenny_amd.checkpoint import quant_from_packed
from qwenny_amd.core import Quant

# The parity bar for bf16 products with f32 accumulation: max |err| <= TOL * RMS(output).
TOL = 2e-2


def make_quant(seed, kind, n, k, group=128):
    """A synthetic stored matrix: kind 'i4' (symmetric), 'i4z' (packed zero points), 'i8' (per-channel int8),
    'i8g' (int8 with a scale per row and `group` columns)."""
    name = f"{kind}_{n}_{k}"
    if kind in ("i8", "i8g"):
        g = group if kind == "i8g" else 0
        t = synth.int8_quant(seed, name, n, k, group=g)
        return quant_from_packed(t["weight_packed"], synth.bf16_to_f32(t["weight_scale"]), 8, g, None,
                                 t["weight_shape"])
    t = synth.int4_quant(seed, name, n, k, zp=kind == "i4z", group=group)
    return quant_from_packed(t["weight_packed"], synth.bf16_to_f32(t["weight_scale"]), 4, group,
                             t.get("weight_zero_point"), t["weight_shape"])


def sub_quant(q, rows):
    """The stored rows `rows` of q as their own Quant (oracle checks on a sample of a large matrix)."""
    rows = np.asarray(rows)
    g = q.cols // q.group
    sc = q.scales.reshape(q.rows, g)[rows]
    of = q.offsets.reshape(q.rows, g)[rows]
    return Quant(q.bits, q.group, len(rows), q.cols, q.q[rows], sc, of)


def oracle_y(q, x):
    """f64 [m][rows] in stored row order."""
    return oracle.gemm_f64(q.bits, q.group, q.q, q.scales, q.offsets, x)


def to_dev(x_bf16):
    import torch

    return torch.from_numpy(np.ascontiguousarray(x_bf16).view(np.int16)).cuda().view(torch.bfloat16)


def dequant_f32(q):
    """The stored matrix dequantized row by row (Quant::row_into), f32 [rows][cols]."""
    return np.stack([q.row_into(r) for r in range(q.rows)])


def emulate_bf16_weights(q, x):
    """What the prefill kernel computes by design: each weight (q - z) s rounded once to bf16, products and sums
    exact (f64 here); per-channel int8 keeps exact integer weights (scale after the sum) and equals the oracle."""
    from qwenny_amd.synth import bf16_to_f32, f32_to_bf16

    w = dequant_f32(q)
    if not (q.bits == 8 and q.group == q.cols):
        w = bf16_to_f32(f32_to_bf16(w))
    return bf16_to_f32(x).astype(np.float64) @ w.astype(np.float64).T


def emulate_f16_operands(q, x):
    """What the prefill kernel computes by design for SwiGLU products of int4 and grouped int8 weights (f16 operands,
    the reference's own): each weight (q - z) s rounded once to f16, the activations converted to f16 (nearest even),
    products and sums exact (f64 here)."""
    from qwenny_amd.synth import bf16_to_f32

    w = dequant_f32(q).astype(np.float16).astype(np.float64)
    xh = bf16_to_f32(x).astype(np.float16).astype(np.float64)
    return xh @ w.T


def emulate_silu_prefill(q, x):
    """The gate or up product as the prefill kernel's SwiGLU launches compute it (f16 operands, but per-channel int8
    exact as in every prefill product)."""
    if q.bits == 8 and q.group == q.cols:
        return emulate_bf16_weights(q, x)
    return emulate_f16_operands(q, x)


def bf16_out_err(got, want):
    """max over outputs of (|got - want| - one bf16 ulp of want) / RMS(want): the error beyond the rounding of a
    bf16 output."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want * want))
    ulp = np.abs(want) * 2.0 ** -8
    return float(np.max(np.maximum(np.abs(got - want) - ulp, 0.0)) / max(rms, 1e-30))


def rel_err(got, want):
    """max |err| / RMS(want)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want * want))
    return float(np.max(np.abs(got - want)) / max(rms, 1e-30))


def silu_bar(got, g, u, tol=TOL):
    """The product bar carried through the SwiGLU epilogue. g and u: the exact gate and up products (f64 [m][rows/2],
    the oracle's); each is allowed max |err| <= tol * RMS, i.e. |dg| <= dg_max = tol RMS(g), |du| <= du_max =
    tol RMS(u), and silu'(v) lies in [-0.0999, 1.0999], so an output computed from products within the bar lies within
    |silu(g)| du_max + 1.1 dg_max (|u| + du_max) of silu(g) u, plus the bf16 rounding of the output (one ulp).
    Returns max over outputs of (|got - silu(g) u| - ulp) / that bound: at most 1 for outputs within the bar."""
    got = np.asarray(got, np.float64)
    g = np.asarray(g, np.float64)
    u = np.asarray(u, np.float64)
    sg = g / (1.0 + np.exp(-g))
    want = sg * u
    dg, du = tol * np.sqrt(np.mean(g * g)), tol * np.sqrt(np.mean(u * u))
    bound = np.abs(sg) * du + 1.1 * dg * (np.abs(u) + du)
    ulp = np.abs(want) * 2.0 ** -8
    return float(np.max(np.maximum(np.abs(got - want) - ulp, 0.0) / bound))
