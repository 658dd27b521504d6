"""The library's launches captured in HIP graphs and replayed: the timing
harness replays every entry point this way, and three of them carry device
state from one launch to the next (the FFN launch's ticket counter and
generation word, the chain's barrier flags).  Each graph is replayed several
times, with other eager work and synchronisations between the replays, and
every replay's bytes must equal the eager launches' bytes.  Nothing in the
library records a memset into a graph: counters are reset by kernels."""
import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()   # fail loudly if the native library is missing
    yield
    torch.cuda.synchronize()


def case(msg):
    print(f"[case] {msg}", flush=True)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def snap(t):
    torch.cuda.synchronize()
    return t.view(torch.uint8).cpu().numpy().copy()


def capture(fn):
    """One eager run on a side stream (default priority), then the capture."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def replay_and_check(g, outs, refs, between, n=4):
    for rep in range(n):
        for t in outs:                                  # poison every output
            t.view(torch.uint8).fill_(0x5A)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, (t, r) in enumerate(zip(outs, refs)):
            assert np.array_equal(snap(t), r), f"replay {rep}: output {i} differs from the eager launch"
        between()                                       # eager work between the replays
        torch.cuda.synchronize()


def test_graph_replays_of_gemv_gemm_and_fused_launches():
    case("graph: GEMV, one-launch Q8_1 + GEMV, fused FWHT GEMV, small-batch and prefill GEMM")
    n_out, n_in = 6144, 5120
    W = dev(O.gen_weights(9100, n_out, n_in))
    x_np = O.gen_normal(9101, n_in)
    x = dev(x_np)
    xq = dev(O.quantize_q8_1(x_np, True))
    X8 = np.stack([O.fwht(O.gen_normal(9102 + t, n_in)) for t in range(8)])
    X300 = np.stack([O.fwht(O.gen_normal(9200 + t, n_in)) for t in range(300)])
    Xq8, Xq300 = dev(O.quantize_chunk_major(X8)), dev(O.quantize_chunk_major(X300))
    ys = [torch.empty(n_out, dtype=torch.float32, device="cuda") for _ in range(3)]
    Y8 = torch.empty(n_out * 8, dtype=torch.float32, device="cuda")
    Y300 = torch.empty(n_out * 300, dtype=torch.float32, device="cuda")

    def launches():
        B.gemv(W, xq, ys[0], n_out, n_in)
        B.quant_gemv(W, x, ys[1], n_out, n_in)
        B.fwht_gemv(W, x, None, ys[2], n_out, n_in)
        B.gemm(W, Xq8, Y8, n_out, n_in, 8)
        B.gemm(W, Xq300, Y300, n_out, n_in, 300)

    outs = ys + [Y8, Y300]
    launches()
    refs = [snap(t) for t in outs]
    g = capture(launches)
    other = torch.empty(n_out, dtype=torch.float32, device="cuda")
    replay_and_check(g, outs, refs, lambda: B.gemv(W, xq, other, n_out, n_in))


@pytest.mark.parametrize("wide,n_out,n_tok", [("2", 600, 300), ("1", 17408, 1024)])
def test_graph_replays_of_wide_prefill_gemm(wide, n_out, n_tok, knobs):
    """The wide prefill kernel in a graph: forced on a ragged shape, and by
    the default rule on a shape it splits into the wide launch and the
    128-row launch for the remaining rows."""
    knobs.set("BONSAI_GEMM_WIDE", wide)
    case(f"graph: prefill GEMM {n_out}x5120x{n_tok}, BONSAI_GEMM_WIDE={wide}")
    n_in = 5120
    W = dev(O.gen_weights(9150, n_out, n_in))
    Xq = dev(O.quantize_chunk_major(O.gen_normal(9151, n_tok * n_in).reshape(n_tok, n_in)))
    Y = torch.empty(n_out * n_tok, dtype=torch.float32, device="cuda")

    def launches():
        B.gemm(W, Xq, Y, n_out, n_in, n_tok)

    launches()
    refs = [snap(Y)]
    g = capture(launches)
    other = torch.empty(n_out * n_tok, dtype=torch.float32, device="cuda")
    replay_and_check(g, [Y], refs, lambda: B.gemm(W, Xq, other, n_out, n_in, n_tok), n=3)


@pytest.mark.parametrize("noalloc", [False, True])
def test_graph_replays_of_ffn_launch(noalloc):
    """Two FFN gate/up launches per graph: the second launch starts from the
    counter the first one left, and every replay from the one before."""
    case(f"graph: FFN gate/up with its glue, noalloc={noalloc}")
    n_ff, n_embd = 17408, 5120
    Wg = dev(O.gen_weights(9300, n_ff, n_embd))
    Wu = dev(O.gen_weights(9301, n_ff, n_embd))
    x1, x2 = dev(O.gen_normal(9302, n_embd)), dev(O.gen_normal(9303, n_embd) * 3)
    nw = dev(O.gen_normal(9304, n_embd) * 0.1 + 1)
    hq1 = torch.empty(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
    hq2 = torch.empty(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
    ws = torch.zeros(B.ffn_workspace_bytes(n_ff), dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")

    def launches():
        for xx, hq in ((x1, hq1), (x2, hq2)):
            if noalloc:
                B.ffn_gate_up_swiglu_noalloc(Wg, Wu, xx, nw, None, None, hq, n_ff, n_embd, 1e-6, status)
            else:
                B.ffn_gate_up_swiglu(Wg, Wu, xx, nw, None, None, hq, n_ff, n_embd, 1e-6, ws, status)

    # eager reference: the separate launches (grouped GEMV, then the glue)
    refs = []
    for xx in (x1, x2):
        g_ = torch.empty(n_ff, dtype=torch.float32, device="cuda")
        u_ = torch.empty(n_ff, dtype=torch.float32, device="cuda")
        B.rmsnorm_fwht_gemv_group([Wg, Wu], xx, nw, None, [g_, u_], [n_ff, n_ff], n_embd, 1e-6)
        ref = torch.empty(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")
        B.swiglu_fwht_quant(g_, u_, None, ref, n_ff)
        refs.append(snap(ref))
    g = capture(launches)
    other = torch.empty(B.q8_bytes(n_ff), dtype=torch.uint8, device="cuda")

    def between():
        B.ffn_gate_up_swiglu(Wg, Wu, x2, nw, None, None, other, n_ff, n_embd, 1e-6, ws, status)

    replay_and_check(g, [hq1, hq2], refs, between)
    assert int(status.item()) == 0, "a finaliser's wait gave up"
    if not noalloc:
        assert snap(ws)[:B.FFN_SYNC_BYTES].view(np.uint32)[0] == 0, "ticket counter not zero"


def test_graph_replays_of_chain():
    """A decode layer as one persistent launch: its barrier flags keep
    counting across replays."""
    case("graph: the decode chain, one layer")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9400)
    from test_gpu_chain import Layer, N_EMBD
    L = Layer(gen, True, 3)
    x0 = torch.randn(N_EMBD, generator=gen, device="cuda")
    r, o = L.buffers(), L.buffers()
    L.separate(x0, r, 1e-6)
    refs = [snap(r[k]) for k in sorted(r)]
    ch = B.Chain(L.steps(x0, o, 1e-6))
    g = capture(ch.run)
    replay_and_check(g, [o[k] for k in sorted(o)], refs, ch.run)
    assert int(ch.status.item()) == 0, "a barrier wait gave up"
