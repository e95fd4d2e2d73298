"""qh_gemm_noalloc, the allocation-free product entry point, against qh_gemm through the C ABI: the same outputs for
every kernel path that uses launch scratch (the argmax table and counter, the prefill's stream-K partials and
counters) and for those that use none, on two calls in a row, the second with a smaller input (the static scratch is
shared between calls and must be left clean by each). Both entry points make the same launch plans, so outputs are
compared bit for bit; the bar of the kernel's arithmetic against the oracle is checked on the first call too."""

import ctypes

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat
from qwenny_amd._lib import check, lib
from qwenny_amd.synth import activations
from tests.helpers import TOL, emulate_bf16_weights, make_quant, oracle_y, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _call(fn, gemm, mat, x, m, y, epi, keys=None, n_out=0, whole=0):
    import torch

    rc = check(fn(gemm._ctx, None, mat._m, _ptr(x), 0, m, None, n_out, _ptr(y), int(epi), _ptr(keys), whole))
    torch.cuda.synchronize()
    return rc


def _both(gemm, mat, x, m, epi, whole=0, n_out=0):
    """(split, y, keys) from qh_gemm and from qh_gemm_noalloc on the same inputs."""
    import torch

    out = []
    for fn in (lib().qh_gemm, lib().qh_gemm_noalloc):
        split = mat.split(m) if epi == Epi.Plain and not whole else 1
        rows = n_out if epi == Epi.Argmax else m
        y = torch.full((split, rows, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
        keys = torch.zeros(max(n_out, 1), dtype=torch.int64, device="cuda") if epi == Epi.Argmax else None
        got = _call(fn, gemm, mat, to_dev(x), m, y, epi, keys, n_out, whole)
        out.append((got, y.cpu().numpy(), None if keys is None else keys.cpu().numpy()))
    return out


# (kind, rows, cols, first m, second m, whole): decode split-K partials (no scratch), stream-K prefill (partials and
# counters), K-sliced and whole-item prefill, and K-sliced prefill below 49 tokens
CASES = [
    ("i4", 6144, 5120, 5, 1, 0),
    ("i4", 4096, 4096, 256, 130, 1),
    ("i4z", 4096, 4096, 256, 130, 1),
    ("i8g", 4096, 4096, 256, 130, 1),
    ("i4", 5120, 17408, 512, 256, 1),
    ("i4", 6144, 5120, 300, 64, 0),
    ("i4", 5120, 17408, 40, 33, 0),
]


@pytest.mark.parametrize("kind,n,k,m1,m2,whole", CASES)
def test_noalloc_plain_matches_gemm(gemm, kind, n, k, m1, m2, whole):
    print(f"no-alloc plain {kind} {n}x{k} m={m1},{m2} whole={whole}", flush=True)
    q = make_quant(900 + m1, kind, n, k)
    mat = Mat.stack(gemm, [q])
    rows = np.sort(np.random.default_rng(m1).choice(n, 64, replace=False))
    for i, m in enumerate((m1, m2)):
        x = activations(910 + i, "x", m, k, outliers=0.01)
        (s_ref, y_ref, _), (s_na, y_na, _) = _both(gemm, mat, x, m, Epi.Plain, whole)
        assert s_ref == s_na
        assert not np.isnan(y_na).any()
        assert np.array_equal(y_ref, y_na), (m, np.abs(y_ref - y_na).max())
        if i == 0:
            from tests.helpers import sub_quant

            sq = sub_quant(q, rows)
            got = y_na.astype(np.float64).sum(0)[:, rows]
            assert rel_err(got, oracle_y(sq, x)) <= TOL
            if mat.kernel(m, whole=whole) == "prefill":
                assert rel_err(got, emulate_bf16_weights(sq, x)) <= 1e-4


@pytest.mark.parametrize("n_out1,n_out2", [(5, 1), (64, 16)])
def test_noalloc_argmax_matches_gemm(gemm, n_out1, n_out2):
    """The argmax table and its counter in the static scratch: keys and logits equal to qh_gemm's on two calls."""
    print(f"no-alloc argmax n_out={n_out1},{n_out2}", flush=True)
    n, k = 65536, 512
    q = make_quant(920, "i4", n, k)
    mat = Mat.stack(gemm, [q])
    for i, n_out in enumerate((n_out1, n_out2)):
        x = activations(921 + i, "x", n_out, k)
        (_, y_ref, k_ref), (_, y_na, k_na) = _both(gemm, mat, x, n_out, Epi.Argmax, n_out=n_out)
        assert np.array_equal(y_ref, y_na)
        assert np.array_equal(k_ref, k_na)
        assert (k_na.view(np.uint64) == oracle.argmax_keys(y_na[0], n)).all()


def test_noalloc_rejects_too_many_argmax_rows(gemm):
    import torch

    from qwenny_amd._lib import QhError

    mat = Mat.stack(gemm, [make_quant(930, "i4", 64, 128)])
    x = to_dev(activations(1, "x", 65, 128))
    y = torch.zeros((65, 64), dtype=torch.float32, device="cuda")
    keys = torch.zeros(65, dtype=torch.int64, device="cuda")
    with pytest.raises(QhError) as e:
        _call(lib().qh_gemm_noalloc, gemm, mat, x, 65, y, Epi.Argmax, keys, 65)
    assert "at most 64" in str(e.value)


def test_noalloc_allocates_nothing(gemm):
    """The property the entry point exists for: a run of calls (decode split-K, stream-K prefill, argmax) leaves the
    device's free memory unchanged (hipMemGetInfo), after one warm-up call per kernel (the runtime loads code objects
    on a kernel's first launch)."""
    import torch

    print("no-alloc memory check", flush=True)
    cases = []
    for kind, n, k, m, epi in (("i4", 6144, 5120, 1, Epi.Plain), ("i4", 4096, 4096, 256, Epi.Plain),
                               ("i4", 65536, 512, 5, Epi.Argmax)):
        mat = Mat.stack(gemm, [make_quant(940 + m, kind, n, k)])
        x = to_dev(activations(941 + m, "x", m, k))
        rows = m
        split = mat.split(m) if epi == Epi.Plain else 1
        y = torch.zeros((split, rows, mat.rows), dtype=torch.float32, device="cuda")
        keys = torch.zeros(m, dtype=torch.int64, device="cuda") if epi == Epi.Argmax else None
        cases.append((mat, x, m, y, epi, keys, m if epi == Epi.Argmax else 0, 1 if m == 256 else 0))

    def run_all():
        for mat, x, m, y, epi, keys, n_out, whole in cases:
            _call(lib().qh_gemm_noalloc, gemm, mat, x, m, y, epi, keys, n_out, whole)

    run_all()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    for _ in range(5):
        run_all()
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, (free0, free1)
