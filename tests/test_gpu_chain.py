"""The decode chain as one persistent launch (bonsai_p40_chain_plan / _run).

Every step must produce the bytes its per-launch entry point produces
(bonsai_p40_rmsnorm_fwht_gemv_group, bonsai_p40_fwht_gemv_group,
bonsai_p40_gemv_group, bonsai_p40_swiglu_fwht_quant), also when a step's input
is an earlier step's output in the same launch (which exercises the grid-wide
barrier: a missed wait reads stale or half-written inputs and changes bits),
over repeated launches on one workspace, and with status staying 0."""
import numpy as np
import pytest

import bonsai_p40 as B
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_EMBD, N_FF, Q_DIM, KV_DIM = 5120, 17408, 6144, 1024


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()   # fail loudly if the native library is missing
    yield
    torch.cuda.synchronize()


def case(msg):
    print(f"[case] {msg}", flush=True)


def weights(gen, n_out, n_in):
    """PQ2_0 rows on the device: codes 0..3 (a few 3s), fp16 scales > 0."""
    nblk = n_out * (n_in // B.QK_PQ2)
    u = torch.rand((nblk, 32, 4), generator=gen, device="cuda")
    codes = torch.where(u <= 0.01, torch.full_like(u, 3.0),
                        torch.clamp(torch.floor((u - 0.01) / (0.99 / 3)), max=2.0)).to(torch.int32)
    packed = (codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)).to(torch.uint8)
    d = (torch.rand((nblk,), generator=gen, device="cuda") * 0.02 + 1e-3).to(torch.float16)
    blocks = torch.empty((nblk, B.PQ2_BYTES), dtype=torch.uint8, device="cuda")
    blocks[:, 0:2] = d.view(torch.uint8).view(nblk, 2)
    blocks[:, 2:] = packed
    return blocks.view(-1)


def signs_vec(seed, n):
    return torch.from_numpy(np.where(O.gen_normal(seed, n) > 0, 1.0, -1.0).astype(np.float32)).cuda()


def f32(n):
    return torch.full((n,), float("nan"), dtype=torch.float32, device="cuda")


def bits(t):
    torch.cuda.synchronize()
    return t.view(torch.int32).cpu().numpy() if t.dtype == torch.float32 else t.cpu().numpy()


class Layer:
    """One decode layer's matrices and the buffers of its outputs."""

    def __init__(self, gen, with_signs, seed):
        self.Wq, self.Wk, self.Wv = (weights(gen, n, N_EMBD) for n in (Q_DIM, KV_DIM, KV_DIM))
        self.Wo = weights(gen, N_EMBD, Q_DIM)
        self.Wg, self.Wu = weights(gen, N_FF, N_EMBD), weights(gen, N_FF, N_EMBD)
        self.Wd = weights(gen, N_EMBD, N_FF)
        self.nw1 = torch.rand(N_EMBD, generator=gen, device="cuda") + 0.5
        self.nw2 = torch.rand(N_EMBD, generator=gen, device="cuda") + 0.5
        s = (lambda k, n: signs_vec(seed * 10 + k, n)) if with_signs else (lambda k, n: None)
        self.s_qkv, self.s_o, self.s_gu, self.s_d = s(1, N_EMBD), s(2, Q_DIM), s(3, N_EMBD), s(4, N_FF)
        self.out = {}

    def buffers(self):
        o = {k: f32(n) for k, n in (("q", Q_DIM), ("k", KV_DIM), ("v", KV_DIM), ("o", N_EMBD), ("g", N_FF),
                                     ("u", N_FF), ("d", N_EMBD))}
        o["hq"] = torch.zeros(B.q8_bytes(N_FF), dtype=torch.uint8, device="cuda")
        return o

    def steps(self, x, o, eps):
        return [
            B.chain_step(B.CHAIN_RMSNORM_FWHT, [self.Wq, self.Wk, self.Wv], [o["q"], o["k"], o["v"]],
                         [Q_DIM, KV_DIM, KV_DIM], N_EMBD, x=x, norm_w=self.nw1, signs=self.s_qkv, eps=eps),
            B.chain_step(B.CHAIN_FWHT, [self.Wo], [o["o"]], [N_EMBD], Q_DIM, x=o["q"], signs=self.s_o),
            B.chain_step(B.CHAIN_RMSNORM_FWHT, [self.Wg, self.Wu], [o["g"], o["u"]], [N_FF, N_FF], N_EMBD,
                         x=o["o"], norm_w=self.nw2, signs=self.s_gu, eps=eps),
            B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=o["g"], x2=o["u"], signs=self.s_d, q_out=o["hq"]),
            B.chain_step(B.CHAIN_Q8, [self.Wd], [o["d"]], [N_EMBD], N_FF, x=o["hq"]),
        ]

    def separate(self, x, o, eps):
        """The same layer as per-step launches (the library's own entry points)."""
        B.rmsnorm_fwht_gemv_group([self.Wq, self.Wk, self.Wv], x, self.nw1, self.s_qkv, [o["q"], o["k"], o["v"]],
                                  [Q_DIM, KV_DIM, KV_DIM], N_EMBD, eps)
        B.fwht_gemv_group([self.Wo], o["q"], self.s_o, [o["o"]], [N_EMBD], Q_DIM)
        B.rmsnorm_fwht_gemv_group([self.Wg, self.Wu], o["o"], self.nw2, self.s_gu, [o["g"], o["u"]],
                                  [N_FF, N_FF], N_EMBD, eps)
        B.swiglu_fwht_quant(o["g"], o["u"], self.s_d, o["hq"], N_FF)
        B.gemv(self.Wd, o["hq"], o["d"], N_EMBD, N_FF)


@pytest.mark.parametrize("with_signs", [False, True])
def test_chain_two_layers_equal_per_step_launches(with_signs):
    case(f"decode chain: 2 layers x 5 steps, signs={with_signs}")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(71 + with_signs)
    layers = [Layer(gen, with_signs, i + 1) for i in range(2)]
    x0 = torch.randn(N_EMBD, generator=gen, device="cuda")
    eps = 1e-6
    ref, got, steps = [], [], []
    x_ref, x_got = x0, x0
    for L in layers:
        r, g = L.buffers(), L.buffers()
        L.separate(x_ref, r, eps)
        steps += L.steps(x_got, g, eps)
        ref.append(r)
        got.append(g)
        x_ref, x_got = r["d"], g["d"]
    ch = B.Chain(steps)
    for launch in range(3):
        for g in got:                        # poison every output
            for k, t in g.items():
                t.fill_(float("nan") if t.dtype == torch.float32 else 0x5A)
        ch.run()
        assert int(ch.status.item()) == 0, "a barrier wait gave up"
        for li, (r, g) in enumerate(zip(ref, got)):
            for k in r:
                assert np.array_equal(bits(g[k]), bits(r[k])), f"launch {launch} layer {li} output {k} differs"
    assert np.all(np.isfinite(bits(ref[-1]["d"]).view(np.float32)))


def test_chain_q8_steps_ragged_groups():
    """Q8 steps on every supported width, groups of 4 with ragged row counts
    (partial 2-row units, one-row matrices), against bonsai_p40_gemv_group."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    steps, checks = [], []
    for n_in, n_outs in ((5120, [1001, 3, 1, 2048]), (6144, [5120, 7, 64, 1]), (17408, [5120, 33])):
        case(f"chain Q8 step n_in={n_in} n_outs={n_outs}")
        Ws = [weights(gen, n, n_in) for n in n_outs]
        x = torch.randn(n_in, generator=gen, device="cuda")
        xq = torch.empty(B.q8_bytes(n_in), dtype=torch.uint8, device="cuda")
        B.fwht_quant(x, None, xq, n_in)
        ys = [f32(n) for n in n_outs]
        refs = [f32(n) for n in n_outs]
        B.gemv_group(Ws, xq, refs, n_outs, n_in)
        steps.append(B.chain_step(B.CHAIN_Q8, Ws, ys, n_outs, n_in, x=xq))
        checks.append((Ws, xq, ys, refs))
    ch = B.Chain(steps)
    ch.run()
    assert int(ch.status.item()) == 0
    for _, _, ys, refs in checks:
        for y, r in zip(ys, refs):
            assert np.array_equal(bits(y), bits(r))


def test_chain_glue_step_alone_and_first():
    """A chain that starts with the SwiGLU glue (no GEMV before it) and one
    that is only the glue, against bonsai_p40_swiglu_fwht_quant."""
    case("chain: glue step first")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(9)
    g = torch.randn(N_FF, generator=gen, device="cuda") * 3
    u = torch.randn(N_FF, generator=gen, device="cuda")
    s = signs_vec(3, N_FF)
    ref = torch.zeros(B.q8_bytes(N_FF), dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(g, u, s, ref, N_FF)
    Wd = weights(gen, N_EMBD, N_FF)
    yref = f32(N_EMBD)
    B.gemv(Wd, ref, yref, N_EMBD, N_FF)
    hq = torch.zeros_like(ref)
    y = f32(N_EMBD)
    for steps in ([B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=g, x2=u, signs=s, q_out=hq)],
                  [B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=g, x2=u, signs=s, q_out=hq),
                   B.chain_step(B.CHAIN_Q8, [Wd], [y], [N_EMBD], N_FF, x=hq)]):
        hq.zero_()
        ch = B.Chain(steps)
        ch.run()
        assert int(ch.status.item()) == 0
        assert np.array_equal(bits(hq), bits(ref))
    assert np.array_equal(bits(y), bits(yref))


def test_chain_gemv_then_glue_only_step():
    """A GEMV step followed by a glue step that ends the chain (the device
    plan's glue-only step after a GEMV), against the per-step launches."""
    case("chain: RMSNorm+FWHT gate/up, then SwiGLU as the last step")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(13)
    Wg, Wu = weights(gen, N_FF, N_EMBD), weights(gen, N_FF, N_EMBD)
    x = torch.randn(N_EMBD, generator=gen, device="cuda")
    nw = torch.rand(N_EMBD, generator=gen, device="cuda") + 0.5
    s_gu, s_d = signs_vec(21, N_EMBD), signs_vec(22, N_FF)
    rg, ru = f32(N_FF), f32(N_FF)
    B.rmsnorm_fwht_gemv_group([Wg, Wu], x, nw, s_gu, [rg, ru], [N_FF, N_FF], N_EMBD, 1e-6)
    rhq = torch.zeros(B.q8_bytes(N_FF), dtype=torch.uint8, device="cuda")
    B.swiglu_fwht_quant(rg, ru, s_d, rhq, N_FF)
    g, u = f32(N_FF), f32(N_FF)
    hq = torch.zeros_like(rhq)
    ch = B.Chain([B.chain_step(B.CHAIN_RMSNORM_FWHT, [Wg, Wu], [g, u], [N_FF, N_FF], N_EMBD, x=x, norm_w=nw,
                               signs=s_gu, eps=1e-6),
                  B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=g, x2=u, signs=s_d, q_out=hq)])
    for launch in range(2):
        hq.zero_()
        ch.run()
        assert int(ch.status.item()) == 0
        assert np.array_equal(bits(g), bits(rg)) and np.array_equal(bits(u), bits(ru))
        assert np.array_equal(bits(hq), bits(rhq)), f"launch {launch}: the glue-only step's bytes differ"


def test_chain_two_glue_steps_in_a_row():
    """gate/up, two SwiGLU glue steps in a row (the second with other signs),
    then the down GEMV on the second one's output, against the per-step
    launches."""
    case("chain: gate/up, SwiGLU, SwiGLU, Q8 down")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(17)
    Wg, Wu = weights(gen, N_FF, N_EMBD), weights(gen, N_FF, N_EMBD)
    Wd = weights(gen, N_EMBD, N_FF)
    x = torch.randn(N_EMBD, generator=gen, device="cuda")
    xq = torch.empty(B.q8_bytes(N_EMBD), dtype=torch.uint8, device="cuda")
    B.fwht_quant(x, None, xq, N_EMBD)
    s1, s2 = signs_vec(31, N_FF), signs_vec(32, N_FF)
    rg, ru, ry = f32(N_FF), f32(N_FF), f32(N_EMBD)
    B.gemv_group([Wg, Wu], xq, [rg, ru], [N_FF, N_FF], N_EMBD)
    rh1 = torch.zeros(B.q8_bytes(N_FF), dtype=torch.uint8, device="cuda")
    rh2 = torch.zeros_like(rh1)
    B.swiglu_fwht_quant(rg, ru, s1, rh1, N_FF)
    B.swiglu_fwht_quant(rg, ru, s2, rh2, N_FF)
    B.gemv(Wd, rh2, ry, N_EMBD, N_FF)
    g, u, y = f32(N_FF), f32(N_FF), f32(N_EMBD)
    h1, h2 = torch.zeros_like(rh1), torch.zeros_like(rh1)
    ch = B.Chain([B.chain_step(B.CHAIN_Q8, [Wg, Wu], [g, u], [N_FF, N_FF], N_EMBD, x=xq),
                  B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=g, x2=u, signs=s1, q_out=h1),
                  B.chain_step(B.CHAIN_SWIGLU, n_in=N_FF, x=g, x2=u, signs=s2, q_out=h2),
                  B.chain_step(B.CHAIN_Q8, [Wd], [y], [N_EMBD], N_FF, x=h2)])
    for launch in range(2):
        for t in (h1, h2):
            t.zero_()
        y.fill_(float("nan"))
        ch.run()
        assert int(ch.status.item()) == 0
        assert np.array_equal(bits(h1), bits(rh1)) and np.array_equal(bits(h2), bits(rh2))
        assert np.array_equal(bits(y), bits(ry)), f"launch {launch}: the down GEMV after two glue steps differs"


def test_chain_barrier_give_up_is_sticky():
    """A launch whose barrier waits cannot succeed ends within about one wait
    bound.  Forced from the host: every workgroup's flag but one says 1000
    barriers passed, so the others wait for a count that workgroup never
    publishes; their bounded waits give up and set the abort word, on which
    every workgroup leaves (every wave exits: nothing spins unbounded).  A
    second launch on that workspace does nothing and counts 1."""
    import time
    case("chain: barrier give-up is sticky (forced from the host)")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(23)
    layer = Layer(gen, False, 5)
    x0 = torch.randn(N_EMBD, generator=gen, device="cuda")
    steps, bufs = [], []                                # bufs keeps every output alive
    for _ in range(4):                                  # 20 steps: about 20 barriers
        bufs.append(layer.buffers())
        steps += layer.steps(x0, bufs[-1], 1e-6)
    ch = B.Chain(steps)
    ch.run()                                             # a good launch first
    torch.cuda.synchronize()
    assert int(ch.status.item()) == 0
    flags = ch.workspace.view(torch.int32)
    n_wg = torch.cuda.get_device_properties(0).multi_processor_count
    flags[:n_wg] = 1000
    flags[3] = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ch.run()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    given_up = int(ch.status.item())
    assert given_up >= 1, "no barrier wait gave up"
    assert int(flags[-1].item()) == 1, "the abort word is not set"
    # one wait bound is some tens of ms; without the abort word every later
    # barrier would poll its full bound again (~20 x that)
    assert dt < 1.0, f"the abandoned launch took {dt:.2f} s"
    ch.run()                                             # the abort word is still set
    torch.cuda.synchronize()
    assert int(ch.status.item()) == given_up + 1
    ch.workspace.zero_()                                 # zero-filled again: launches work
    ch.status.zero_()
    ch.run()
    torch.cuda.synchronize()
    assert int(ch.status.item()) == 0
