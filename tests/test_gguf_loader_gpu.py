"""GPU: the PQ2_0 loader (p40-kernel_amd/gguf_pq2.py load_pq2) on synthetic
GGUF files, then the GEMVs on the loaded weights through the C ABI.

Bars: arena bytes equal the file's bytes (native layout) or the oracle's
repack of them (repack layout), exactly; GEMV outputs within 1e-5 normwise of
the oracle on the file's bytes and bit-identical to the same launch on a
freshly uploaded copy.
"""
import sys

import numpy as np
import pytest

import bonsai_p40 as B
import gguf_pq2 as G
import gguf_synth as S
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-5

# widths of the model's projections; rows cut down so the file stays small
SHAPES = [("blk.0.attn_qkv.weight", 5120, 96), ("blk.0.ssm_out.weight", 6144, 40),
          ("blk.0.ffn_down.weight", 17408, 24), ("blk.3.attn_k.weight", 5120, 33)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    B.lib()
    yield
    torch.cuda.synchronize()


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def normwise(got, ref):
    scale = max(float(np.max(np.abs(ref))), 1e-30)
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64)))) / scale


@pytest.fixture(scope="module")
def model_file(tmp_path_factory):
    rng = np.random.default_rng(77)
    payload = {name: S.random_pq2(rng, n_out, n_in) for name, n_in, n_out in SHAPES}
    norm = rng.standard_normal(5120).astype(np.float32)
    ts = [("blk.0.attn_norm.weight", (5120,), S.F32, norm.tobytes())]
    ts += [(name, (n_in, n_out), S.PQ2, payload[name]) for name, n_in, n_out in SHAPES]
    # 32-byte file alignment: the arena has to re-align every tensor
    path = tmp_path_factory.mktemp("gguf") / "synthetic.gguf"
    path.write_bytes(S.build([("general.alignment", S.T_U32, 32)], ts, alignment=32))
    return str(path), payload, norm


@pytest.mark.parametrize("staging", [1 << 20, 4096])
def test_load_native_bytes_and_gemv(model_file, staging):
    path, payload, _ = model_file
    case(f"load_pq2 native staging={staging}")
    wts = G.load_pq2(path, layout="native", staging_bytes=staging)
    assert len(wts) == len(SHAPES)
    for name, n_in, n_out in SHAPES:
        t = wts[name]
        assert (t.n_in, t.n_out, t.layout) == (n_in, n_out, "native")
        assert t.data.data_ptr() % G.ARENA_ALIGN == 0
        W = np.frombuffer(payload[name], np.uint8)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(t.data.cpu().numpy(), W)
        x = O.gen_normal(900 + n_in, n_in)
        xq = O.quantize_q8_1(x, True)
        xqd = torch.from_numpy(xq).cuda()
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(t.data, xqd, y, n_out, n_in)
        Wd = torch.from_numpy(W.copy()).cuda()
        y2 = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv(Wd, xqd, y2, n_out, n_in)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert normwise(got, O.gemv(W, xq, n_out, n_in)) <= TOL
        np.testing.assert_array_equal(got.view(np.uint32), y2.cpu().numpy().view(np.uint32))


def test_load_repack_bytes_and_gemv(model_file):
    path, payload, _ = model_file
    case("load_pq2 repack")
    wts = G.load_pq2(path, layout="repack", staging_bytes=64 << 10)
    for name, n_in, n_out in SHAPES:
        t = wts[name]
        assert t.layout == "repack"
        W = np.frombuffer(payload[name], np.uint8)
        torch.cuda.synchronize()
        Wr = t.data.cpu().numpy()
        np.testing.assert_array_equal(Wr, O.repack(W, n_out, n_in))
        x = O.gen_normal(950 + n_in, n_in) * 1.3
        y = torch.full((n_out,), float("nan"), dtype=torch.float32, device="cuda")
        B.gemv_repack(t.data, torch.from_numpy(x).cuda(), y, n_out, n_in)
        torch.cuda.synchronize()
        assert normwise(y.cpu().numpy(), O.gemv_repack(Wr, x, n_out, n_in)) <= TOL


def test_load_selected_and_norm(model_file):
    path, payload, norm = model_file
    case("load_pq2 names= + load_tensor")
    names = ["blk.0.ffn_down.weight", "blk.3.attn_k.weight"]
    wts = G.load_pq2(path, names=names)
    assert sorted(wts.tensors) == sorted(names)
    assert [wts[n].arena_offset for n in names] == [0, (24 * 136 * 34 + 255) // 256 * 256]
    torch.cuda.synchronize()
    for n in names:
        np.testing.assert_array_equal(wts[n].data.cpu().numpy(), np.frombuffer(payload[n], np.uint8))
    nw = G.load_tensor(path, "blk.0.attn_norm.weight")
    assert nw.is_cuda and nw.shape == (5120,)
    np.testing.assert_array_equal(nw.cpu().numpy(), norm)
