"""Parity of the HIP products with the oracle (dequantize-then-matmul in f64), through the C ABI.

Bar: max |err| <= 2e-2 * RMS(output) (bf16 operands, f32 accumulation); bf16 outputs (SwiGLU) may differ by one
more bf16 ulp of the value. Beyond the bar, each kernel is pinned to its own arithmetic: the skinny kernel multiplies
exact integers by bf16 activations and applies scales in f32, so it matches the f64 oracle to 1e-4; the prefill kernel
rounds each dequantized weight (q - z) s to bf16 once, so it matches an f64 product of bf16-rounded weights to 1e-4
(per-channel int8 keeps exact integer weights and matches the oracle itself).
"""

import numpy as np
import pytest

import oracle
from qwenny_amd import SKINNY_MAX_M, Epi, Mat, Wt, row_order
from qwenny_amd.synth import activations, bf16_to_f32
from tests.helpers import (TOL, bf16_out_err, emulate_bf16_weights, emulate_silu_prefill, make_quant, oracle_y, rel_err,
                           silu_bar, sub_quant, to_dev)

pytestmark = pytest.mark.gpu

# i8: int8 per channel (exact integer prefill); i8g: int8 with a scale per row and 128 columns (the reference's
# default load mode, dequantized per group in the prefill kernel)
KINDS = ["i4", "i4z", "i8", "i8g"]
WT_OF = {"i4": Wt.I4, "i4z": Wt.I4Z, "i8": Wt.I8, "i8g": Wt.I8}


def _plain(gemm, mat, x, m, stream=None):
    import torch

    split = mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    got = gemm.run(stream, m, mat, to_dev(x), y, Epi.Plain)
    torch.cuda.synchronize()
    assert got == split
    return y.sum(0).cpu().numpy().astype(np.float64)


def _check(got, q, x, kernel):
    """The bar against the oracle, and the arithmetic of the kernel that ran (Mat.kernel) to 1e-4."""
    want = oracle_y(q, x)
    err = rel_err(got, want)
    assert err <= TOL, f"max|err|/rms {err:.3e} vs the oracle"
    exact = want if kernel == "skinny" else emulate_bf16_weights(q, x)
    err = rel_err(got, exact)
    assert err <= 1e-4, f"max|err|/rms {err:.3e} vs the kernel's arithmetic"


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16])
def test_skinny_plain(gemm, kind, m):
    print(f"skinny plain {kind} m={m}", flush=True)
    q = make_quant(11 + m, kind, 512, 1024)
    x = activations(5 + m, "x", m, 1024)
    mat = Mat.stack(gemm, [q])
    assert mat.wt == WT_OF[kind]
    assert mat.per_channel == (kind == "i8")
    _check(_plain(gemm, mat, x, m), q, x, mat.kernel(m))


@pytest.mark.parametrize("kind", ["i4", "i4z", "i8", "i8g"])
@pytest.mark.parametrize("m", [1, 2, 5])
@pytest.mark.parametrize("rows,cols", [(16, 512), (48, 512), (80, 1024), (400, 2560)])
def test_decode_odd_tiles(gemm, kind, m, rows, cols):
    """Decode products of 1, 3, 5 and 25 tiles (the last wave of a pair holding one tile), with 4-group and one-group
    waves: the lean decode kernels' edges, and int8's one-tile waves at 1-2 tokens. Each output against the oracle;
    the returned split matches Mat.split."""
    print(f"decode odd tiles {kind} m={m} {rows}x{cols}", flush=True)
    q = make_quant(60 + rows + m, kind, rows, cols)
    x = activations(61 + m, "x", m, cols)
    mat = Mat.stack(gemm, [q])
    got = _plain(gemm, mat, x, m)
    assert rel_err(got, oracle_y(q, x)) <= 1e-4


@pytest.mark.parametrize("kind", ["i4", "i4z"])
@pytest.mark.parametrize("half,cols", [(24, 512), (40, 2560), (8, 6144)])
def test_silu_decode_odd_tiles(gemm, kind, half, cols):
    """One-token SwiGLU over 3, 5 and 1 tiles of [gate; up], K of 4, 20 and 48 groups (the lean one-token SwiGLU
    kernel takes K of at most 16 chunks of 4 groups; 48 groups go to skinny_kernel): against the oracle."""
    import torch

    print(f"silu decode odd tiles {kind} half={half} cols={cols}", flush=True)
    gate, up = make_quant(70 + half, kind, half, cols), make_quant(71 + half, kind, half, cols)
    x = activations(72, "x", 1, cols)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    y = torch.full((1, half), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, 1, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    want = oracle.silu_glu(np.concatenate([oracle_y(gate, x), oracle_y(up, x)], axis=1), None)
    assert bf16_out_err(got, want) <= 1e-4


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [17, 33, 48, 49, 64, 130, 256, 300])
def test_prefill_plain(gemm, kind, m):
    print(f"prefill plain {kind} m={m}", flush=True)
    q = make_quant(21 + m, kind, 384, 768)
    x = activations(6 + m, "x", m, 768, outliers=0.01)
    mat = Mat.stack(gemm, [q])
    assert mat.per_channel == (kind == "i8")
    _check(_plain(gemm, mat, x, m), q, x, mat.kernel(m))


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("m", [1, 5, 40, 300])
def test_silu(gemm, kind, m):
    """SwiGLU epilogue: bf16 silu(gate) * up over the interleaved [gate; up] tiles. For decode sizes the products are
    exact, so the output matches the oracle within the bar (plus the bf16 rounding of the output); for prefill sizes
    the inputs of the epilogue carry the bf16 rounding of each weight (held to the bar in test_prefill_plain), and the
    epilogue is checked against silu over the same arithmetic."""
    import torch

    print(f"silu {kind} m={m}", flush=True)
    n, k = 512, 512
    gate = make_quant(31, kind, n // 2, k)
    up = make_quant(32, kind, n // 2, k)
    x = activations(7, "x", m, k)
    mat = Mat.stack(gemm, [gate, up], silu=True)
    y = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Silu) == 1
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    if mat.kernel(m, Epi.Silu) == "skinny":
        full = np.concatenate([oracle_y(gate, x), oracle_y(up, x)], axis=1)
        tol = TOL
    else:
        full = np.concatenate([emulate_silu_prefill(gate, x), emulate_silu_prefill(up, x)], axis=1)
        tol = 1e-3
    want = oracle.silu_glu(full, row_order(n, True))
    assert bf16_out_err(got, want) <= tol
    # every kernel also against the oracle's exact dequantize-then-matmul: at the product bar carried through the
    # epilogue, and within the bar of the output itself
    g, u = oracle_y(gate, x), oracle_y(up, x)
    assert silu_bar(got, g, u) <= 1.0
    assert bf16_out_err(got, oracle.silu_glu(np.concatenate([g, u], axis=1), None)) <= TOL


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n_out", [1, 3, 16, 40])
def test_argmax(gemm, kind, n_out):
    import torch

    print(f"argmax {kind} n_out={n_out}", flush=True)
    n, k, steps = 1024, 512, 50
    q = make_quant(41, kind, n, k)
    x = activations(8, "x", steps, k)
    rows = np.random.default_rng(3).choice(steps, n_out, replace=False).astype(np.int32)
    mat = Mat.stack(gemm, [q])
    y = torch.zeros((n_out, n), dtype=torch.float32, device="cuda")
    keys = torch.zeros(n_out, dtype=torch.int64, device="cuda")
    out_rows = torch.from_numpy(rows).cuda()
    gemm.run(None, steps, mat, to_dev(x), y, Epi.Argmax, out_rows=out_rows, n_out=n_out, keys=keys)
    torch.cuda.synchronize()
    want = oracle_y(q, x[rows])
    got = y.cpu().numpy()
    assert rel_err(got, want) <= TOL
    # the keys are exactly those of the logits the kernel wrote
    assert (keys.cpu().numpy().view(np.uint64) == oracle.argmax_keys(got, n)).all()
    assert (np.argmax(want, axis=1) == np.argmax(got, axis=1)).all()


def test_skinny_baseline_shape(gemm):
    """M=1, K=2560, N=9728, symmetric."""
    q = make_quant(1, "i4", 9728, 2560)
    x = activations(1, "x", 1, 2560)
    mat = Mat.stack(gemm, [q])
    assert rel_err(_plain(gemm, mat, x, 1), oracle_y(q, x)) <= 1e-4


@pytest.mark.parametrize("n_out", [1, 5, 16, 64])
def test_argmax_many_workgroups_repeated(gemm, n_out):
    """Thousands of workgroups folding their maxima through the argmax scratch table, several launches in a row with
    different activations: each launch's keys must be exactly those of its own logits (the table is left clean)."""
    import torch

    print(f"argmax many n_out={n_out}", flush=True)
    n, k = 65536, 256
    q = make_quant(43, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    for rep in range(3):
        x = activations(60 + rep, "x", n_out, k)
        y = torch.zeros((n_out, n), dtype=torch.float32, device="cuda")
        keys = torch.zeros(n_out, dtype=torch.int64, device="cuda")
        gemm.run(None, n_out, mat, to_dev(x), y, Epi.Argmax, n_out=n_out, keys=keys)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert (keys.cpu().numpy().view(np.uint64) == oracle.argmax_keys(got, n)).all(), rep
        assert rel_err(got, oracle_y(q, x)) <= TOL


@pytest.mark.parametrize("kind", ["i4", "i4z", "i8g"])
def test_argmax_running_key(gemm, kind):
    """keys[] is a running maximum (the caller clears it; products of one step may add to it): a launch leaves
    max(keys[t], its own best key). One token over 65,536 rows (thousands of workgroups), the caller's key set just
    below, just above, and far below the launch's best."""
    import torch

    print(f"argmax running key {kind}", flush=True)
    n, k = 65536, 512
    q = make_quant(47, kind, n, k)
    mat = Mat.stack(gemm, [q])
    x = to_dev(activations(71, "x", 1, k))
    y = torch.zeros((1, n), dtype=torch.float32, device="cuda")

    def run(init):
        keys = torch.tensor([np.int64(np.uint64(init).view(np.int64))], dtype=torch.int64, device="cuda")
        gemm.run(None, 1, mat, x, y, Epi.Argmax, n_out=1, keys=keys)
        torch.cuda.synchronize()
        return int(keys.cpu().numpy().view(np.uint64)[0])

    best = run(0)
    got = y.cpu().numpy()
    assert best == int(oracle.argmax_keys(got, n)[0])
    tenth = int(oracle.argmax_keys(np.sort(got, axis=1)[:, :-9], n - 9)[0])  # a key of a lower logit
    assert tenth < best
    assert run(best - 1) == best
    assert run(best + 1) == best + 1
    assert run(tenth) == best
    assert run(0) == best


def test_kernel_switch_large_int4(gemm):
    """Split-K plain and SwiGLU products of 33-48 tokens on int4 and grouped int8 matrices of at least 2^26 weights run
    on the prefill kernel (faster there); 32 tokens, whole products, the argmax, per-channel int8 and a matrix one
    group of K short of 2^26 weights stay on the skinny kernel. Each side matches its own arithmetic (64 sampled rows
    of 4096 x 16384 matrices, symmetric int4 and with zero points; a [gate; up] SwiGLU product of 2 x 2048 rows)."""
    n, k = 4096, 16384
    q = make_quant(180, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    assert [mat.kernel(m) for m in (1, 32, 33, 48, 49)] == ["skinny", "skinny", "prefill", "prefill", "prefill"]
    assert mat.kernel(40, whole=True) == "skinny" and mat.kernel(40, Epi.Argmax) == "skinny"
    assert mat.kernel(40, Epi.Silu) == "prefill" and mat.kernel(32, Epi.Silu) == "skinny"
    assert Mat.stack(gemm, [make_quant(181, "i4", n, k - 128)]).kernel(40) == "skinny"
    assert Mat.stack(gemm, [make_quant(183, "i8", n, k)]).kernel(40) == "skinny"
    assert Mat.stack(gemm, [make_quant(184, "i8g", n, k)]).kernel(40) == "prefill"
    qz = make_quant(182, "i4z", n, k)
    zmat = Mat.stack(gemm, [qz])
    assert zmat.kernel(40) == "prefill"
    rows = np.sort(np.random.default_rng(3).choice(n, 64, replace=False))
    sq = sub_quant(q, rows)
    for m in (33, 48):
        print(f"kernel switch zero points m={m}", flush=True)
        x = activations(190 + m, "x", m, k, outliers=0.01)
        _check(_plain(gemm, zmat, x, m)[:, rows], sub_quant(qz, rows), x, zmat.kernel(m))
    import torch

    gate, up = make_quant(185, "i4", n // 2, k), make_quant(186, "i4", n // 2, k)
    gu = Mat.stack(gemm, [gate, up], silu=True)
    half = np.sort(np.random.default_rng(4).choice(n // 2, 32, replace=False))
    for m in (32, 40):
        print(f"kernel switch SwiGLU m={m}", flush=True)
        x = activations(195 + m, "x", m, k)
        y = torch.full((m, n // 2), float("nan"), dtype=torch.bfloat16, device="cuda")
        assert gemm.run(None, m, gu, to_dev(x), y, Epi.Silu) == 1
        torch.cuda.synchronize()
        # output column j is silu(gate row j) * up row j
        sg, su = sub_quant(gate, half), sub_quant(up, half)
        if gu.kernel(m, Epi.Silu) == "skinny":
            g, u, tol = oracle_y(sg, x), oracle_y(su, x), TOL
        else:
            g, u, tol = emulate_silu_prefill(sg, x), emulate_silu_prefill(su, x), 1e-3
        want = oracle.silu_glu(np.concatenate([g, u], axis=1), None)
        assert bf16_out_err(y.float().cpu().numpy()[:, half], want) <= tol
        # both kernels against the oracle's exact product at the bar
        eg, eu = oracle_y(sg, x), oracle_y(su, x)
        assert silu_bar(y.float().cpu().numpy()[:, half], eg, eu) <= 1.0
        assert bf16_out_err(y.float().cpu().numpy()[:, half], oracle.silu_glu(np.concatenate([eg, eu], 1), None)) <= TOL
    for m in (32, 33, 48):
        print(f"kernel switch m={m}", flush=True)
        x = activations(183 + m, "x", m, k, outliers=0.01)
        split = mat.split(m)
        got = _plain(gemm, mat, x, m)[:, rows]
        _check(got, sq, x, mat.kernel(m))
        assert m == 32 or 1 < split <= 16
        if m == 33:  # the whole product on the skinny kernel: one partial, the split product's value
            y = torch.full((1, m, n), float("nan"), dtype=torch.float32, device="cuda")
            assert gemm.run_split(None, m, mat, to_dev(x), y, Epi.Plain, True) == 1
            torch.cuda.synchronize()
            _check(y[0].cpu().numpy().astype(np.float64)[:, rows], sq, x, "skinny")


def test_argmax_rejects_too_many_rows(gemm):
    import torch

    from qwenny_amd._lib import QhError

    q = make_quant(44, "i4", 64, 128)
    mat = Mat.stack(gemm, [q])
    x = to_dev(activations(1, "x", 65, 128))
    y = torch.zeros((65, 64), dtype=torch.float32, device="cuda")
    keys = torch.zeros(65, dtype=torch.int64, device="cuda")
    with pytest.raises(QhError):
        gemm.run(None, 65, mat, x, y, Epi.Argmax, n_out=65, keys=keys)


def test_prefill_rejects_x_past_32bit_offsets(gemm):
    """Above SKINNY_MAX_M tokens the prefill kernel addresses x's rows with 32-bit byte offsets: a row stride that
    puts the last token past 4 GiB is refused before any launch."""
    import torch

    from qwenny_amd._lib import QhError

    m = SKINNY_MAX_M + 1
    mat = Mat.stack(gemm, [make_quant(45, "i4", 64, 128)])
    x = torch.zeros((m, 128), dtype=torch.bfloat16, device="cuda")
    y = torch.zeros((m, 64), dtype=torch.float32, device="cuda")
    ldx = 1 << 26  # (m - 1) * ldx * 2 bytes = 6 GiB
    assert (m - 1) * ldx * 2 > 1 << 32
    with pytest.raises(QhError) as e:
        gemm.run(None, m, mat, x, y, Epi.Plain, ldx=ldx)
    assert "4 GiB" in str(e.value)


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("n,k", [(16, 128), (48, 384), (80, 640), (272, 1152)])
def test_small_and_odd_shapes(gemm, kind, n, k):
    """Edge shapes at both kernels' boundaries: a single tile and a single group; tile counts that leave a wave's or a
    prefill workgroup's last tiles past the matrix (3, 5 and 17 tiles); group counts that are not a multiple of 4
    (one group per decode wave); token counts on both sides of the skinny/prefill switch and a 130-token step."""
    for m in (1, 3, 16, 17, 48, 49, 130):
        print(f"odd shape {kind} {n}x{k} m={m}", flush=True)
        q = make_quant(170 + m, kind, n, k)
        x = activations(171 + m, "x", m, k, outliers=0.01)
        mat = Mat.stack(gemm, [q])
        _check(_plain(gemm, mat, x, m), q, x, mat.kernel(m))
