"""Products captured into a HIP graph, as the engine captures its decode step (src/cuda/core.rs:1151-1192): the
launches allocate nothing and clear nothing with memsets, and the argmax table and the stream-K item counters return
to zero inside the kernels, so every replay must give the eager results. The graph is replayed several times with new
activations and eager launches between replays; each replay is checked against an eager run on the same inputs."""

import numpy as np
import pytest

import oracle
from qwenny_amd import Epi, Mat
from qwenny_amd.synth import activations
from tests.helpers import make_quant, to_dev

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gemm):
    import torch

    print("graph replays", flush=True)
    k = 4096
    dec = Mat.stack(gemm, [make_quant(91, "i4", 2048, k)])       # skinny, split-K partials
    head = Mat.stack(gemm, [make_quant(92, "i4z", 8192, k)])     # skinny, argmax across workgroups
    pre = Mat.stack(gemm, [make_quant(93, "i4", 4096, k)])       # prefill at 256 tokens: items spread (stream-K)
    sl = Mat.stack(gemm, [make_quant(94, "i4", 1024, k)])        # prefill at 64 tokens: K-sliced partials
    big = Mat.stack(gemm, [make_quant(95, "i4", 16384, k)])      # 2^26 weights at 40 tokens: prefill, K-sliced
    m_dec, m_pre, m_sl, m_big = 1, 256, 64, 40
    assert sl.split(m_sl) > 1 and big.kernel(m_big) == "prefill" and big.split(m_big) > 1
    y_big = torch.empty((big.split(m_big), m_big, big.rows), dtype=torch.float32, device="cuda")
    x_dec = torch.empty((m_dec, k), dtype=torch.bfloat16, device="cuda")
    x_pre = torch.empty((m_pre, k), dtype=torch.bfloat16, device="cuda")
    y_sl = torch.empty((sl.split(m_sl), m_sl, sl.rows), dtype=torch.float32, device="cuda")
    split = dec.split(m_dec)
    y_dec = torch.empty((split, m_dec, dec.rows), dtype=torch.float32, device="cuda")
    y_head = torch.empty((m_dec, head.rows), dtype=torch.float32, device="cuda")
    keys = torch.zeros(m_dec, dtype=torch.int64, device="cuda")
    y_pre = torch.empty((pre.split(m_pre), m_pre, pre.rows), dtype=torch.float32, device="cuda")

    def step(stream):
        gemm.run(stream, m_dec, dec, x_dec, y_dec, Epi.Plain)
        gemm.run(stream, m_dec, head, x_dec, y_head, Epi.Argmax, n_out=m_dec, keys=keys)
        gemm.run(stream, m_pre, pre, x_pre, y_pre, Epi.Plain)
        gemm.run(stream, m_sl, sl, x_pre, y_sl, Epi.Plain)  # the first 64 tokens of x_pre
        gemm.run(stream, m_big, big, x_pre, y_big, Epi.Plain)  # the first 40

    def outputs():
        return y_dec.sum(0).cpu().numpy(), y_head.cpu().numpy(), keys.cpu().numpy().view(np.uint64).copy(), \
            y_pre.cpu().numpy(), y_sl.cpu().numpy(), y_big.cpu().numpy()

    def load_inputs(seed):
        x_dec.copy_(to_dev(activations(seed, "x", m_dec, k)))
        x_pre.copy_(to_dev(activations(seed + 1, "x", m_pre, k)))
        keys.zero_()  # the caller clears keys before a step (embed does in the reference), a fill kernel here

    load_inputs(1)
    step(None)  # first launches outside the capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step(s)
    torch.cuda.synchronize()
    for rep in range(4):
        load_inputs(10 + 2 * rep)
        torch.cuda.synchronize()
        step(None)  # eager
        torch.cuda.synchronize()
        want = outputs()
        keys.zero_()
        y_dec.fill_(float("nan"))
        y_head.fill_(float("nan"))
        y_pre.fill_(float("nan"))
        y_sl.fill_(float("nan"))
        y_big.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = outputs()
        for a, b in zip(got, want):
            assert np.array_equal(a, b), rep
        assert (got[2] == oracle.argmax_keys(got[1], head.rows)).all(), rep


def test_empty_step_launches_nothing(gemm):
    """n = 0 tokens: the product returns split 1 and touches nothing (the reference's empty-step path)."""
    import torch

    mat = Mat.stack(gemm, [make_quant(94, "i4", 256, 512)])
    x = torch.zeros((1, 512), dtype=torch.bfloat16, device="cuda")
    y = torch.full((1, 256), 7.0, dtype=torch.float32, device="cuda")
    assert gemm.run(None, 0, mat, x, y, Epi.Plain) == 1
    torch.cuda.synchronize()
    assert (y.cpu().numpy() == 7.0).all()


def test_graph_consumers_replay(gemm):
    """The partials consumers and the LoRA epilogue captured after a decode product (add_rmsnorm's spread sum and
    norm, sum_parts, lora_add, lora_silu), replayed with new partials: every replay equals the eager launches."""
    import torch

    from qwenny_amd import add_rmsnorm, lora_add, lora_silu, sum_parts

    print("graph replays of the consumers", flush=True)
    m, hid, split, rank, gu = 3, 5120, 34, 16, 1024
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.empty(split, m, hid, device="cuda")
    h0 = torch.randn(m, hid, device="cuda", generator=g)
    h = torch.empty_like(h0)
    w = torch.rand(hid, device="cuda", generator=g) + 0.5
    y = torch.empty(m, hid, dtype=torch.bfloat16, device="cuda")
    s = torch.empty(m, hid, device="cuda")
    xa = torch.empty(2, m, 32, device="cuda")
    b = (torch.randn(gu, rank, device="cuda", generator=g) * 0.05).half().view(torch.int16)
    tab = torch.tensor([512, 2**31 - 1, 2**31 - 1, 2**31 - 1, 0, 16, -1, -1], dtype=torch.int32, device="cuda")
    tab_silu = torch.tensor([2**31 - 1] * 4 + [0, 16, -1, -1], dtype=torch.int32, device="cuda")
    slot = torch.tensor([0, 1, 0], dtype=torch.int32, device="cuda")
    scale = torch.tensor([0.5, 0.0], device="cuda")
    ygu = torch.empty(m, gu, device="cuda")
    ylo = torch.empty(m, gu, device="cuda")
    mid = torch.empty(m, gu // 2, dtype=torch.bfloat16, device="cuda")

    def step():
        h.copy_(h0)
        add_rmsnorm(None, h, x, split, m, hid, w, y)
        sum_parts(None, x, split, m, hid, s)
        lora_add(None, xa, 2, 32, b, rank, gu, tab, slot, scale, m, ylo)
        lora_silu(None, xa, 2, 32, b, rank, gu, tab_silu, slot, scale, m, ygu, mid)

    def load(seed):
        gg = torch.Generator(device="cuda").manual_seed(seed)
        x.copy_(torch.randn(split, m, hid, device="cuda", generator=gg) * 0.3)
        xa.copy_(torch.randn(2, m, 32, device="cuda", generator=gg))
        ygu.copy_(torch.randn(m, gu, device="cuda", generator=gg))
        ylo.copy_(torch.randn(m, gu, device="cuda", generator=gg))

    outs = lambda: [t.float().cpu().numpy().copy() for t in (h, y, s, ylo, mid)]
    load(1)
    step()
    torch.cuda.synchronize()
    graph, st = torch.cuda.CUDAGraph(), torch.cuda.Stream()
    with torch.cuda.stream(st):
        with torch.cuda.graph(graph, stream=st):
            step()
    torch.cuda.synchronize()
    for rep in range(3):
        load(10 + rep)
        ylo_in = ylo.clone()
        torch.cuda.synchronize()
        step()
        torch.cuda.synchronize()
        want = outs()
        ylo.copy_(ylo_in)
        for t in (y, s, mid):
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for a, b_ in zip(outs(), want):
            assert np.array_equal(a, b_), rep


def test_abi_graph_capture_replays(gemm):
    """The library's own capture entry points (qh_graph_begin / end / launch / free, through qwenny_amd.Graph) over a
    step that also holds the whole-row decode kernels (one and five tokens), the one-token SwiGLU product and the
    prefill SwiGLU product with its f16 activation conversion: every replay, with new inputs and eager launches
    between replays, equals the eager step bit for bit."""
    import torch

    from qwenny_amd import Graph
    from qwenny_amd._lib import QhError

    print("graph capture through the C ABI", flush=True)
    k = 5120
    dec = Mat.stack(gemm, [make_quant(96, "i4", 2048, k)])
    gu_q = [make_quant(97, "i4", 1024, k), make_quant(98, "i4z", 1024, k)]
    gu = Mat.stack(gemm, gu_q, silu=True)
    x1 = torch.empty((1, k), dtype=torch.bfloat16, device="cuda")
    x5 = torch.empty((256, k), dtype=torch.bfloat16, device="cuda")
    y_w1 = torch.empty((1, dec.rows), dtype=torch.float32, device="cuda")
    y_w5 = torch.empty((5, dec.rows), dtype=torch.float32, device="cuda")
    y_s1 = torch.empty((1, gu.rows // 2), dtype=torch.bfloat16, device="cuda")
    y_s256 = torch.empty((256, gu.rows // 2), dtype=torch.bfloat16, device="cuda")
    outs = (y_w1, y_w5, y_s1, y_s256)

    def step(stream):
        assert gemm.run_split(stream, 1, dec, x1, y_w1, Epi.Plain, True) == 1
        assert gemm.run_split(stream, 5, dec, x5, y_w5, Epi.Plain, True) == 1
        gemm.run(stream, 1, gu, x1, y_s1, Epi.Silu)
        gemm.run(stream, 256, gu, x5, y_s256, Epi.Silu)

    def load(seed):
        x1.copy_(to_dev(activations(seed, "x", 1, k)))
        x5.copy_(to_dev(activations(seed + 1, "x", 256, k)))

    load(1)
    step(None)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with pytest.raises(QhError):
        Graph.capture(0, lambda: None)  # the null stream cannot be captured
    g = Graph.capture(s, lambda: step(s))
    try:
        for rep in range(3):
            load(20 + 2 * rep)
            torch.cuda.synchronize()
            step(None)
            torch.cuda.synchronize()
            want = [t.float().cpu().numpy().copy() for t in outs]
            for t in outs:
                t.fill_(float("nan"))
            torch.cuda.synchronize()
            g.launch(s)
            s.synchronize()
            got = [t.float().cpu().numpy() for t in outs]
            for a, b in zip(got, want):
                assert np.array_equal(a, b), rep
    finally:
        g.close()
