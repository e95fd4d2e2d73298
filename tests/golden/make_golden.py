"""Writes tests/golden/mlx_affine.npz: known-answer vectors from the closed-form generator of the reference's own
kernel test (src/mlx/metal.rs:375-384) — x = f16(((i * 17) % 101 - 50) / 53), q words i * 7919 + 0x1949abcd,
sc = f16((i % 11 + 1) / 97), bi = f16(-8 sc) — with the expected products from that test's f64 loop
(src/mlx/metal.rs:393-403), evaluated here with numpy. The activations are rounded to bf16 (the build's activation
type) before the products; the expected values use the same rounded activations.

Run: python tests/golden/make_golden.py
"""

import os

import numpy as np


def mlx_case(m, n, k, group, bits):
    """The generator's inputs: x f16 [m][k], q u32 [n][k * bits / 32], sc and bi f16 [n][k / group]."""
    pack = 32 // bits
    i = np.arange(m * k)
    x = (((i * 17) % 101).astype(np.float32) - 50.0) / 53.0
    x16 = x.astype(np.float16).reshape(m, k)
    wi = np.arange(n * k // pack, dtype=np.uint64)
    q = ((wi * 7919 + 0x1949ABCD) & 0xFFFFFFFF).astype(np.uint32).reshape(n, k // pack)
    si = np.arange(n * k // group)
    sc = ((si % 11 + 1).astype(np.float32) / 97.0).astype(np.float16).reshape(n, k // group)
    bi = (-8.0 * sc.astype(np.float32)).astype(np.float16)
    return x16, q, sc, bi


def expected(x16, q, sc, bi, group, bits):
    """The reference test's f64 triple loop, vectorised: sum_d x[r][d] (qi sc[g] + bi[g])."""
    from qwenny_amd.synth import bf16_to_f32, f32_to_bf16

    m, k = x16.shape
    n = q.shape[0]
    pack = 32 // bits
    d = np.arange(k)
    qi = ((q[:, d // pack] >> ((d % pack) * bits).astype(np.uint32)) & ((1 << bits) - 1)).astype(np.float64)
    g = d // group
    w = qi * sc.astype(np.float64)[:, g] + bi.astype(np.float64)[:, g]
    xb = f32_to_bf16(x16.astype(np.float32))
    return xb, bf16_to_f32(xb).astype(np.float64) @ w.T


# the shapes of src/mlx/metal.rs:373-382
SHAPES = [(3, 35, 128, 64, 4), (5, 64, 256, 128, 4), (8, 33, 128, 128, 4), (16, 32, 64, 64, 4), (8, 35, 256, 128, 8),
          (5, 64, 1024, 128, 4), (5, 48, 1024, 128, 4), (1, 35, 1024, 128, 4)]


def main():
    import sys

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))))
    out = {"count": np.array(len(SHAPES))}
    for i, (m, n, k, group, bits) in enumerate(SHAPES):
        x16, q, sc, bi = mlx_case(m, n, k, group, bits)
        xb, y = expected(x16, q, sc, bi, group, bits)
        out.update({f"xb{i}": xb, f"q{i}": q, f"sc{i}": sc.astype(np.float32), f"bi{i}": bi.astype(np.float32),
                    f"y{i}": y, f"bits{i}": np.array(bits), f"group{i}": np.array(group),
                    f"shape{i}": np.array([m, n, k])})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "mlx_affine.npz")
    np.savez_compressed(path, **out)
    print("wrote", path)


if __name__ == "__main__":
    main()
