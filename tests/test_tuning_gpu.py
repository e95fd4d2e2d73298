"""The tuning overrides of the decode partition, read once per context at qh_open, give the products of the default
partition: K-wave rows within a workgroup (QH_SKINNY_PLAIN_WK, plain partials reduced through LDS before the staged
16-byte stores) and forced tile waves (QH_SKINNY_TILE_WAVES). Token counts cover one and two 16-token blocks (the
two-block kernel takes at most 512 threads per workgroup, so K-wave rows beyond that bound fall back to the default
partition). Sums of the partials are checked against the default context's to f32 rounding of the different split
(the split itself changes), and against the oracle at the product bar."""

import numpy as np
import pytest

from qwenny_amd import Epi, Gemm, Mat
from qwenny_amd.synth import activations
from tests.helpers import make_quant, oracle_y, rel_err, to_dev

pytestmark = pytest.mark.gpu


def _sum(gemm, mat, x, m):
    import torch

    split = mat.split(m)
    y = torch.full((split, m, mat.rows), float("nan"), dtype=torch.float32, device="cuda")
    assert gemm.run(None, m, mat, to_dev(x), y, Epi.Plain) == split
    torch.cuda.synchronize()
    got = y.cpu().numpy().astype(np.float64)
    assert not np.isnan(got).any()
    return got.sum(0), split


@pytest.mark.parametrize("env", [{"QH_SKINNY_PLAIN_WK": "2"}, {"QH_SKINNY_PLAIN_WK": "4"},
                                 {"QH_SKINNY_TILE_WAVES": "4"}, {"QH_SKINNY_TILE_WAVES": "8"}])
@pytest.mark.parametrize("m", [1, 5, 17, 33])
def test_tuned_partition_matches_default(gemm, monkeypatch, env, m):
    print(f"tuned partition {env} m={m}", flush=True)
    for k_, v in env.items():
        monkeypatch.setenv(k_, v)
    tuned = Gemm.load(0)  # reads the overrides
    try:
        q = make_quant(900 + m, "i4", 1024, 4096)
        x = activations(901 + m, "x", m, 4096)
        want_sum, _ = _sum(gemm, Mat.stack(gemm, [q]), x, m)
        got_sum, _ = _sum(tuned, Mat.stack(tuned, [q]), x, m)
        assert rel_err(got_sum, want_sum) <= 1e-5
        assert rel_err(got_sum, oracle_y(q, x)) <= 1e-4
    finally:
        tuned.close()


@pytest.mark.parametrize("pk", ["2", "4"])
def test_part_len_covers_tuned_split(monkeypatch, pk):
    """Under QH_SKINNY_PLAIN_WK the skinny split depends on the token count; part_len must cover the largest
    split x tokens over every count (a product into a part_len-sized buffer writes no further)."""
    import torch

    print(f"part_len QH_SKINNY_PLAIN_WK={pk}", flush=True)
    monkeypatch.setenv("QH_SKINNY_PLAIN_WK", pk)
    tuned = Gemm.load(0)
    try:
        q = make_quant(950, "i4", 1024, 4096)
        mat = Mat.stack(tuned, [q])
        max_tok = 48
        need = max(mat.split(m) * m * mat.rows for m in range(1, max_tok + 1))
        n = tuned.part_len([mat], max_tok)
        assert n >= need
        # a product of every token count into a buffer of exactly part_len floats, guarded by a canary after it
        y = torch.full((n + 4096,), float("nan"), dtype=torch.float32, device="cuda")
        for m in (1, 2, 3, 4, 16, 17, 33, 48):
            x = activations(951 + m, "x", m, 4096)
            split = tuned.run(None, m, mat, to_dev(x), y, Epi.Plain)
            assert split * m * mat.rows <= n
        torch.cuda.synchronize()
        assert torch.isnan(y[n:]).all()
    finally:
        tuned.close()
