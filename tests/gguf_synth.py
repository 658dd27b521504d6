"""Writer of synthetic GGUF files for the loader tests.

Written from the GGUF v3 layout (magic, version, tensor count, key/value
count, key/values, tensor infos, padding to ``general.alignment``, data) and
kept independent of the reader under test: it shares no code with it.  The
shipped Ternary-Bonsai-2-27B file is not available offline, so
``bonsai27b_header`` builds its tensor list and key/values (the geometry
tools/check_gguf.py:23-67 expects) with no tensor data behind them.
"""
import struct

import numpy as np

T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_FMT = {T_U8: "B", T_I8: "b", T_U16: "H", T_I16: "h", T_U32: "I", T_I32: "i", T_F32: "f",
        T_BOOL: "?", T_U64: "Q", T_I64: "q", T_F64: "d"}

PQ2, F32, F16 = 142, 0, 1


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t: int, v) -> bytes:
    if t == T_STR:
        return _str(v)
    if t == T_ARR:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    return struct.pack("<" + _FMT[t], v)


def tensor_nbytes(dims, ttype) -> int:
    n = 1
    for d in dims[1:]:
        n *= d
    if ttype == PQ2:
        return dims[0] // 128 * 34 * n
    return dims[0] * n * {F32: 4, F16: 2}[ttype]


def build(kvs, tensors, alignment=32, with_data=True, version=3) -> bytes:
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml type, payload
    bytes or None)].  Payloads of None are zero-filled (with_data) or left out
    (header only).  Each tensor's data starts on ``alignment``."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _val(t, v)
    off, datas = 0, []
    for name, dims, tt, payload in tensors:
        n = tensor_nbytes(dims, tt)
        if payload is not None and len(payload) != n:
            raise ValueError(f"{name}: payload {len(payload)} bytes, dims need {n}")
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", tt, off)
        datas.append((off, payload if payload is not None else bytes(n)))
        off = (off + n + alignment - 1) // alignment * alignment
    if not with_data:
        return head
    pad = (-len(head)) % alignment
    out = bytearray(head + bytes(pad))
    base = len(out)
    out += bytes(off)
    for o, p in datas:
        out[base + o:base + o + len(p)] = p
    return bytes(out)


def bonsai27b_kvs(**override):
    kv = [
        ("general.architecture", T_STR, "qwen35"),
        ("general.name", T_STR, "synthetic"),
        ("qwen35.block_count", T_U32, 64),
        ("qwen35.context_length", T_U32, 262144),
        ("qwen35.embedding_length", T_U32, 5120),
        ("qwen35.feed_forward_length", T_U32, 17408),
        ("qwen35.attention.head_count", T_U32, 24),
        ("qwen35.attention.head_count_kv", T_U32, 4),
        ("qwen35.attention.key_length", T_U32, 256),
        ("qwen35.attention.value_length", T_U32, 256),
        ("qwen35.attention.layer_norm_rms_epsilon", T_F32, 1e-6),
        ("qwen35.full_attention_interval", T_U32, 4),
        ("qwen35.ssm.conv_kernel", T_U32, 4),
        ("qwen35.ssm.state_size", T_U32, 128),
        ("qwen35.ssm.group_count", T_U32, 16),
        ("qwen35.ssm.time_step_rank", T_U32, 48),
        ("qwen35.ssm.inner_size", T_U32, 6144),
        ("qwen35.rope.dimension_count", T_U32, 64),
        ("prism.hadamard.block_size", T_U32, 1024),
        ("prism.hadamard.transform", T_STR, "normalized-sylvester-walsh-hadamard"),
        ("prism.hadamard.axis", T_STR, "input-last-dimension"),
        ("tokenizer.ggml.tokens", T_ARR, (T_STR, ["<a>", "b", "c"])),
        ("tokenizer.ggml.scores", T_ARR, (T_F32, [0.0, -1.0, -2.0])),
        ("general.alignment", T_U32, 32),
    ]
    out = []
    for k, t, v in kv:
        if k in override:
            ov = override[k]
            if ov is None:
                continue                      # key removed
            t, v = ov
        out.append((k, t, v))
    return out


def bonsai27b_tensors():
    """The 27B tensor list: 64 layers, every 4th one full attention."""
    ts = [("token_embd.weight", (5120, 248320), PQ2, None),
          ("output_norm.weight", (5120,), F32, None),
          ("output.weight", (5120, 248320), PQ2, None)]
    for il in range(64):
        p = f"blk.{il}."
        ts.append((p + "attn_norm.weight", (5120,), F32, None))
        if (il + 1) % 4 == 0:
            ts += [(p + "attn_q.weight", (5120, 12288), PQ2, None),
                   (p + "attn_k.weight", (5120, 1024), PQ2, None),
                   (p + "attn_v.weight", (5120, 1024), PQ2, None),
                   (p + "attn_output.weight", (6144, 5120), PQ2, None),
                   (p + "attn_q_norm.weight", (256,), F32, None)]
        else:
            ts += [(p + "attn_qkv.weight", (5120, 10240), PQ2, None),
                   (p + "attn_gate.weight", (5120, 6144), PQ2, None),
                   (p + "ssm_out.weight", (6144, 5120), PQ2, None),
                   (p + "ssm_a", (48,), F32, None),
                   (p + "ssm_conv1d.weight", (4, 10240), F32, None)]
        ts += [(p + "post_attention_norm.weight", (5120,), F32, None),
               (p + "ffn_gate.weight", (5120, 17408), PQ2, None),
               (p + "ffn_up.weight", (5120, 17408), PQ2, None),
               (p + "ffn_down.weight", (17408, 5120), PQ2, None)]
    return ts


def bonsai27b_header(kv_override=None, tensors=None) -> bytes:
    return build(bonsai27b_kvs(**(kv_override or {})),
                 bonsai27b_tensors() if tensors is None else tensors, with_data=False)


def random_pq2(rng: np.random.Generator, n_out: int, n_in: int) -> bytes:
    """Ternary PQ2_0 blocks with positive fp16 scales in about [0.004, 0.06)."""
    nblk = n_out * (n_in // 128)
    b = np.empty((nblk, 34), np.uint8)
    d = (rng.uniform(0.004, 0.06, nblk)).astype(np.float16).view(np.uint8).reshape(nblk, 2)
    codes = rng.integers(0, 3, (nblk, 32, 4), dtype=np.uint8)
    b[:, :2] = d
    b[:, 2:] = codes[..., 0] | (codes[..., 1] << 2) | (codes[..., 2] << 4) | (codes[..., 3] << 6)
    return b.tobytes()
