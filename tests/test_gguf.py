"""CPU: GGUF header reader, the 27B geometry check and the loader's host-side
checks (p40-kernel_amd/gguf_pq2.py).

The shipped model file is not available offline; the check is exercised on
the full 27B tensor list written as a header-only synthetic file
(tests/gguf_synth.py) and on planted mistakes, each of which must produce
exactly the failure the reference tool's decision rules give
(tools/check_gguf.py:123-173).
"""
import struct

import numpy as np
import pytest

import gguf_pq2 as G
import gguf_synth as S


def _fails(data: bytes):
    h = G.read_header(data, partial=True)
    return G.check_geometry(h)[0]


# ---------------------------------------------------------------- reader
def test_header_known_answer():
    """A header assembled byte by byte: values, alignment and data offset."""
    raw = b"GGUF" + struct.pack("<IQQ", 3, 1, 3)
    raw += struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<II", 4, 64)
    raw += struct.pack("<Q", 4) + b"name" + struct.pack("<IQ", 8, 3) + b"abc"
    raw += struct.pack("<Q", 3) + b"arr" + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<iii", 1, -2, 3)
    raw += struct.pack("<Q", 1) + b"w" + struct.pack("<IQQ", 2, 256, 2) + struct.pack("<IQ", 142, 0)
    h = G.read_header(raw)
    assert h.version == 3 and h.n_tensors == 1
    assert h.kv["general.alignment"] == 64 and h.alignment == 64
    assert h.kv["name"] == "abc"
    arr = h.kv["arr"]
    assert arr.elem_type == G.KV_I32 and arr.count == 3
    assert list(arr.values()) == [1, -2, 3]
    t = h.tensors[0]
    assert (t.name, t.dims, t.type, t.offset) == ("w", (256, 2), 142, 0)
    assert t.nbytes == 2 * 2 * 34
    assert h.data_offset == (len(raw) + 63) // 64 * 64


def test_every_kv_type_round_trips():
    kvs = [("u8", S.T_U8, 250), ("i8", S.T_I8, -7), ("u16", S.T_U16, 65000), ("i16", S.T_I16, -300),
           ("u32", S.T_U32, 4000000000), ("i32", S.T_I32, -5), ("f32", S.T_F32, 0.5),
           ("b", S.T_BOOL, True), ("s", S.T_STR, "héllo"), ("u64", S.T_U64, 2 ** 40),
           ("i64", S.T_I64, -2 ** 40), ("f64", S.T_F64, 0.1),
           ("as", S.T_ARR, (S.T_STR, ["x", "", "yz"])),
           ("af", S.T_ARR, (S.T_F64, [1.5, -2.25])),
           ("aa", S.T_ARR, (S.T_ARR, [(S.T_U8, [1, 2]), (S.T_U8, [])]))]
    h = G.read_header(S.build(kvs, []))
    for k, t, v in kvs:
        assert h.kv_types[k] == t
        if t == S.T_ARR:
            got = h.kv[k].values()
            if v[0] == S.T_ARR:
                assert [list(a.values()) for a in got] == [list(a[1]) for a in v[1]]
            else:
                assert list(got) == list(v[1])
        elif t == S.T_F32:
            assert h.kv[k] == np.float32(v)
        else:
            assert h.kv[k] == v
    assert h.tensors == [] and h.data_offset % 32 == 0


def test_tensor_offsets_and_sizes():
    ts = [("a", (256, 3), S.PQ2, None), ("b", (5,), S.F32, None), ("c", (7, 2), S.F16, None)]
    data = S.build([("general.alignment", S.T_U32, 64)], ts, alignment=64)
    h = G.read_header(data)
    assert [t.nbytes for t in h.tensors] == [204, 20, 28]
    assert [t.offset for t in h.tensors] == [0, 256, 320]
    assert h.data_offset % 64 == 0
    assert h.data_offset + 320 + ((28 + 63) // 64) * 64 == len(data)
    assert [t.generic_name for t in h.tensors] == ["a", "b", "c"]
    assert G.TensorInfo("blk.12.ffn_up.weight", (1,), 0, 0).generic_name == "blk.X.ffn_up.weight"


def test_bad_magic_version_and_alignment():
    good = S.build([], [])
    with pytest.raises(G.GGUFError, match="magic"):
        G.read_header(b"GGUX" + good[4:])
    with pytest.raises(G.GGUFError, match="version 1"):
        G.read_header(S.build([], [], version=1))
    with pytest.raises(G.GGUFError, match="alignment"):
        G.read_header(S.build([("general.alignment", S.T_U32, 48)], []))
    with pytest.raises(G.GGUFError, match="alignment"):
        G.read_header(S.build([("general.alignment", S.T_U64, 64)], []))
    with pytest.raises(G.GGUFError, match="unknown key/value type"):
        G.read_header(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k"
                      + struct.pack("<I", 13))


def test_truncated_header():
    full = S.bonsai27b_header()
    h = G.read_header(full)
    assert len(h.tensors) == len(S.bonsai27b_tensors()) and h.truncated is None
    cut = full[:len(full) * 2 // 3]
    with pytest.raises(G.GGUFTruncated):
        G.read_header(cut)
    hp = G.read_header(cut, partial=True)
    assert hp.truncated and hp.data_offset is None
    assert 0 < len(hp.tensors) < len(h.tensors)
    assert hp.tensors == h.tensors[:len(hp.tensors)]
    # the key/values must be whole even for a partial download
    with pytest.raises(G.GGUFTruncated):
        G.read_header(full[:200], partial=True)
    # a cut list fails the counted groups (fewer layers than the engine needs)
    fails = G.check_geometry(hp)[0]
    assert any("group blk.X.attn_norm.weight " in f for f in fails)
    assert not any(f.startswith("metadata key") for f in fails)
    assert G.check_loadable(hp, len(cut)) == [f"tensor list incomplete: {hp.truncated}"]


# ---------------------------------------------------------------- the check
def test_full_27b_geometry_passes():
    h = G.read_header(S.bonsai27b_header())
    fails, rep = G.check_geometry(h)
    assert fails == []
    assert sum(1 for r in rep if r.startswith("  [pass]")) == len(G.EXPECT_KV) + len(G.EXPECT_TENSORS)
    assert not any(r.startswith("  [FAIL]") for r in rep)
    assert rep[-1].startswith("multi-token-prediction tensors: none")


def _mutate_tensors(fn):
    return [x for x in (fn(t) for t in S.bonsai27b_tensors()) if x is not None]


def _set(name, dims=None, tt=None):
    def f(t):
        if t[0] != name:
            return t
        return (t[0], dims if dims is not None else t[1], tt if tt is not None else t[2], None)
    return f


PLANTED = {
    "kv value": (dict(kv_override={"qwen35.block_count": (S.T_U32, 63)}), ["qwen35.block_count"]),
    "kv string": (dict(kv_override={"general.architecture": (S.T_STR, "llama")}),
                  ["general.architecture"]),
    "kv missing": (dict(kv_override={"prism.hadamard.axis": None}), ["prism.hadamard.axis"]),
    # a u64-stored value is not read (the tool decodes u32, i32 and strings only)
    "kv u64": (dict(kv_override={"qwen35.embedding_length": (S.T_U64, 5120)}),
               ["qwen35.embedding_length"]),
    "kv i32 accepted": (dict(kv_override={"qwen35.ssm.state_size": (S.T_I32, 128)}), []),
    "down transposed": (dict(tensors=_mutate_tensors(
        lambda t: (t[0], (5120, 17408), t[2], None) if t[0].endswith("ffn_down.weight") else t)),
        ["blk.X.ffn_down.weight"]),
    "k as f16": (dict(tensors=_mutate_tensors(
        lambda t: (t[0], t[1], S.F16, None) if t[0].endswith("attn_k.weight") else t)),
        ["blk.X.attn_k.weight"]),
    "one qkv missing": (dict(tensors=_mutate_tensors(
        lambda t: None if t[0] == "blk.0.attn_qkv.weight" else t)), ["blk.X.attn_qkv.weight"]),
    "output rows": (dict(tensors=_mutate_tensors(_set("output.weight", dims=(5120, 248321)))),
                    ["output.weight"]),
    # one layer's norm off: its own group fails and the 63 left fail the count
    "one norm wide": (dict(tensors=_mutate_tensors(_set("blk.5.attn_norm.weight", dims=(5121,)))),
                      ["blk.X.attn_norm.weight", "blk.X.attn_norm.weight"]),
    # an uncounted group may have any number of layers
    "one up missing": (dict(tensors=_mutate_tensors(
        lambda t: None if t[0] == "blk.3.ffn_up.weight" else t)), []),
    "mtp block": (dict(tensors=S.bonsai27b_tensors() + [("blk.64.nextn.eh_proj.weight", (10240, 5120),
                                                          S.PQ2, None)]), ["nextn"]),
    # tensors the engine does not check are ignored
    "extra tensor": (dict(tensors=S.bonsai27b_tensors() + [("rope_freqs.weight", (32,), S.F32, None)]),
                     []),
}


@pytest.mark.parametrize("name", list(PLANTED))
def test_planted_mistakes(name):
    kw, want = PLANTED[name]
    fails = _fails(S.bonsai27b_header(**kw))
    assert len(fails) == len(want), fails
    for f, w in zip(sorted(fails), sorted(want)):
        assert w in f, (f, w)


def test_cli(tmp_path, capsys):
    p = tmp_path / "head.bin"
    p.write_bytes(S.bonsai27b_header())
    assert G.main([str(p)]) == 0
    assert "usable: every key and tensor group matches" in capsys.readouterr().out
    assert G.main(["--header", str(p)]) == 0
    capsys.readouterr()
    p.write_bytes(S.bonsai27b_header(kv_override={"qwen35.block_count": (S.T_U32, 32)}))
    assert G.main([str(p)]) == 1
    out = capsys.readouterr().out
    assert "not usable by this engine: 1 problem" in out
    assert "metadata key qwen35.block_count is 32; the engine is built for 64" in out
    p.write_bytes(b"NOPE" + bytes(20))
    assert G.main([str(p)]) == 1
    assert G.main([]) == 2


# ------------------------------------------------------ the loader, host side
def _small_file(alignment=32):
    rng = np.random.default_rng(5)
    ts = [("blk.0.ffn_up.weight", (1024, 3), S.PQ2, S.random_pq2(rng, 3, 1024)),
          ("blk.0.attn_norm.weight", (5,), S.F32, np.arange(5, dtype=np.float32).tobytes()),
          ("small.weight", (640, 2), S.PQ2, S.random_pq2(rng, 2, 640)),
          ("cube.weight", (1024, 2, 1), S.PQ2, S.random_pq2(rng, 2, 1024))]
    return S.build([("general.alignment", S.T_U32, alignment)], ts, alignment=alignment)


def test_check_loadable():
    data = _small_file()
    h = G.read_header(data)
    assert G.check_loadable(h, len(data)) == []
    # the repack kernel works on 8-block groups: n_in = 640 is 5 blocks
    probs = G.check_loadable(h, len(data), layout="repack")
    assert len(probs) == 1 and probs[0].startswith("small.weight") and "1024" in probs[0]
    assert G.check_loadable(h, len(data), names=["blk.0.ffn_up.weight", "cube.weight"],
                            layout="repack") == []
    assert "not PQ2_0" in G.check_loadable(h, len(data), names=["blk.0.attn_norm.weight"])[0]
    with pytest.raises(KeyError):
        G.check_loadable(h, len(data), names=["nope"])
    # data past the end of a cut file
    probs = G.check_loadable(h, len(data) - 40)
    assert len(probs) == 1 and "ends at byte" in probs[0]


def test_check_loadable_rejects_bad_offsets_and_dims():
    raw = b"GGUF" + struct.pack("<IQQ", 3, 2, 0)
    raw += struct.pack("<Q", 1) + b"a" + struct.pack("<IQQ", 2, 1024, 1) + struct.pack("<IQ", 142, 8)
    raw += struct.pack("<Q", 1) + b"b" + struct.pack("<IQQQ", 3, 1024, 1, 2) + struct.pack("<IQ", 142, 512)
    h = G.read_header(raw)
    probs = G.check_loadable(h, 1 << 20)
    assert any(p.startswith("a:") and "aligned" in p for p in probs)
    assert any(p.startswith("b:") and "2-D" in p for p in probs)


def test_plan_arena():
    h = G.read_header(_small_file())
    sel = [t for t in h.tensors if t.type == G.GGML_TYPE_PQ2_0]
    offs, total = G.plan_arena(sel)
    # 816, 340 and 544 bytes in 1024-, 512- and 768-byte slots
    assert offs == [0, 1024, 1536]
    assert total == 1536 + 768
    assert all(o % G.ARENA_ALIGN == 0 for o in offs)


def test_load_rejects_before_touching_a_device(tmp_path):
    p = tmp_path / "m.gguf"
    p.write_bytes(_small_file())
    with pytest.raises(ValueError, match="layout"):
        G.load_pq2(str(p), device="cpu", layout="tiled")
    with pytest.raises(ValueError, match="staging"):
        G.load_pq2(str(p), device="cpu", staging_bytes=1000)
    with pytest.raises(G.GGUFError, match="geometry check failed"):
        G.load_pq2(str(p), device="cpu", check=True)
    with pytest.raises(G.GGUFError, match="not loadable"):
        G.load_pq2(str(p), device="cpu", names=["blk.0.attn_norm.weight"])
