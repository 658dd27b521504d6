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
