"""GGUF header reader, Bonsai-27B geometry check and PQ2_0 weight loader.

Three layers, each usable alone:

* ``read_header(buf)`` parses a GGUF v2/v3 header (key/values and tensor
  infos) from any buffer -- a whole file through ``mmap`` or only the first
  megabytes of a download.  Nothing is copied: arrays stay views into the
  buffer.
* ``check_geometry(header)`` makes the decisions of the reference tool
  tools/check_gguf.py:97-180 against its tables (:23-67): every expected
  key/value, the (n_in, n_out, type) and per-layer count of each tensor
  group, and the refusal of files that carry an MTP/nextn block.
  ``python gguf_pq2.py [--header] FILE`` prints the report and exits 0 (all
  checks pass), 1 (a check failed) or 2 (usage), as the reference tool does.
* ``load_pq2(path, ...)`` is the loader the reference's repack notes ask for
  (docs/REPACK.md:96-99, 121-124): every PQ2_0 tensor is streamed from the
  file through two pinned staging buffers into ONE device arena (256-byte
  aligned slots, so every tensor meets the streaming GEMV's 16-byte
  alignment), optionally converted to the aligned repack layout by
  ``bonsai_p40_repack`` on the way in.  Peak device memory is the arena plus,
  for the repack layout, one buffer the size of the largest tensor.

PQ2_0 is ggml type 142 (check_gguf.py:17): blocks of 128 weights in 34 bytes,
ne0 = n_in (the contiguous axis), ne1 = n_out.
"""
from __future__ import annotations

import mmap
import os
import re
import struct
import sys
from dataclasses import dataclass, field

import numpy as np

GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_BF16 = 30
GGML_TYPE_PQ2_0 = 142

# bytes per block and elements per block of the types this path reads
_TYPE_BLOCK = {GGML_TYPE_F32: (4, 1), GGML_TYPE_F16: (2, 1), GGML_TYPE_BF16: (2, 1),
               GGML_TYPE_PQ2_0: (34, 128)}

GGUF_MAGIC = b"GGUF"
GGUF_DEFAULT_ALIGNMENT = 32
ARENA_ALIGN = 256

# GGUF key/value type ids
KV_U8, KV_I8, KV_U16, KV_I16, KV_U32, KV_I32, KV_F32, KV_BOOL = range(8)
KV_STRING, KV_ARRAY, KV_U64, KV_I64, KV_F64 = range(8, 13)
_KV_SCALAR = {KV_U8: "<u1", KV_I8: "<i1", KV_U16: "<u2", KV_I16: "<i2", KV_U32: "<u4",
              KV_I32: "<i4", KV_F32: "<f4", KV_BOOL: "<u1", KV_U64: "<u8", KV_I64: "<i8",
              KV_F64: "<f8"}
_KV_FMT = {KV_U8: "<B", KV_I8: "<b", KV_U16: "<H", KV_I16: "<h", KV_U32: "<I", KV_I32: "<i",
           KV_F32: "<f", KV_BOOL: "<B", KV_U64: "<Q", KV_I64: "<q", KV_F64: "<d"}

# ---- the geometry the engine is built for (tools/check_gguf.py:23-67) -------
# These tables have to be the reference's numbers: they describe the shipped
# Ternary-Bonsai-2-27B file, which both engines consume unchanged.
EXPECT_KV = {
    "general.architecture": "qwen35",
    "qwen35.block_count": 64,
    "qwen35.embedding_length": 5120,
    "qwen35.feed_forward_length": 17408,
    "qwen35.attention.head_count": 24,
    "qwen35.attention.head_count_kv": 4,
    "qwen35.attention.key_length": 256,
    "qwen35.attention.value_length": 256,
    "qwen35.full_attention_interval": 4,
    "qwen35.ssm.conv_kernel": 4,
    "qwen35.ssm.state_size": 128,
    "qwen35.ssm.group_count": 16,
    "qwen35.ssm.time_step_rank": 48,
    "qwen35.ssm.inner_size": 6144,
    "qwen35.rope.dimension_count": 64,
    "prism.hadamard.block_size": 1024,
    "prism.hadamard.transform": "normalized-sylvester-walsh-hadamard",
    "prism.hadamard.axis": "input-last-dimension",
}

# layer-generic tensor name -> (n_in, n_out or None for "any", ggml type)
EXPECT_TENSORS = {
    "output.weight": (5120, 248320, GGML_TYPE_PQ2_0),
    "token_embd.weight": (5120, 248320, GGML_TYPE_PQ2_0),
    "blk.X.attn_norm.weight": (5120, None, GGML_TYPE_F32),
    "blk.X.post_attention_norm.weight": (5120, None, GGML_TYPE_F32),
    "blk.X.ffn_down.weight": (17408, 5120, GGML_TYPE_PQ2_0),
    "blk.X.ffn_gate.weight": (5120, 17408, GGML_TYPE_PQ2_0),
    "blk.X.ffn_up.weight": (5120, 17408, GGML_TYPE_PQ2_0),
    "blk.X.attn_qkv.weight": (5120, 10240, GGML_TYPE_PQ2_0),       # 48 linear-attention layers
    "blk.X.attn_gate.weight": (5120, 6144, GGML_TYPE_PQ2_0),
    "blk.X.ssm_out.weight": (6144, 5120, GGML_TYPE_PQ2_0),
    "blk.X.attn_q.weight": (5120, 12288, GGML_TYPE_PQ2_0),         # 16 full-attention layers
    "blk.X.attn_k.weight": (5120, 1024, GGML_TYPE_PQ2_0),
    "blk.X.attn_v.weight": (5120, 1024, GGML_TYPE_PQ2_0),
    "blk.X.attn_output.weight": (6144, 5120, GGML_TYPE_PQ2_0),
}

# tensor groups whose number of layers is fixed
TENSOR_COUNT = {"blk.X.attn_qkv.weight": 48, "blk.X.attn_q.weight": 16,
                "blk.X.attn_k.weight": 16, "blk.X.attn_v.weight": 16,
                "blk.X.attn_output.weight": 16, "blk.X.attn_gate.weight": 48,
                "blk.X.ssm_out.weight": 48, "blk.X.attn_norm.weight": 64}

# key/value types whose values the check reads (check_gguf.py:114-118); a
# checked key stored as any other type reads as absent and fails
_CHECKED_KV_TYPES = (KV_U32, KV_I32, KV_STRING)

_MTP_RE = re.compile(r"nextn|mtp|draft|eagle", re.I)
_LAYER_RE = re.compile(r"blk\.\d+\.")


class GGUFError(ValueError):
    """Malformed or unsupported GGUF content."""


class GGUFTruncated(GGUFError):
    """The buffer ends inside the header."""


@dataclass(frozen=True)
class KVArray:
    """A GGUF array value, left in the buffer: ``elem_type``, ``count`` and
    the byte span [start, end) of its elements.  ``values()`` decodes it."""
    buf: object
    elem_type: int
    count: int
    start: int
    end: int

    def values(self):
        if self.elem_type in _KV_SCALAR:
            return np.frombuffer(self.buf, dtype=_KV_SCALAR[self.elem_type],
                                 count=self.count, offset=self.start)
        cur = _Cursor(self.buf, self.start)
        return [cur.value(self.elem_type) for _ in range(self.count)]


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dims: tuple          # ggml order: dims[0] = ne0 (contiguous), dims[1] = ne1, ...
    type: int
    offset: int          # relative to the data section

    @property
    def generic_name(self) -> str:
        return _LAYER_RE.sub("blk.X.", self.name)

    @property
    def nbytes(self) -> int | None:
        """Bytes of the tensor's data, or None for a type this path does not know."""
        tb = _TYPE_BLOCK.get(self.type)
        if tb is None or not self.dims:
            return None
        size, per = tb
        if self.dims[0] % per:
            return None
        n = self.dims[0] // per * size
        for d in self.dims[1:]:
            n *= d
        return n


@dataclass
class GGUFHeader:
    version: int
    n_tensors: int
    kv: dict = field(default_factory=dict)          # key -> decoded value (arrays as KVArray)
    kv_types: dict = field(default_factory=dict)    # key -> GGUF type id
    tensors: list = field(default_factory=list)     # TensorInfo, file order
    alignment: int = GGUF_DEFAULT_ALIGNMENT
    data_offset: int | None = None                  # None when the tensor list is cut off
    truncated: str | None = None                    # why the tensor list is incomplete

    def tensor(self, name: str) -> TensorInfo:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)


class _Cursor:
    __slots__ = ("b", "o", "n")

    def __init__(self, buf, off: int = 0):
        self.b = buf
        self.o = off
        self.n = len(buf)

    def take(self, fmt: str):
        size = struct.calcsize(fmt)
        if self.o + size > self.n:
            raise GGUFTruncated(f"header ends at byte {self.n}, needs {self.o + size}")
        v = struct.unpack_from(fmt, self.b, self.o)
        self.o += size
        return v[0] if len(v) == 1 else v

    def string(self) -> str:
        n = self.take("<Q")
        if self.o + n > self.n:
            raise GGUFTruncated(f"string of {n} bytes at {self.o} passes the end ({self.n})")
        s = bytes(self.b[self.o:self.o + n]).decode("utf-8", "replace")
        self.o += n
        return s

    def value(self, t: int):
        if t in _KV_SCALAR:
            v = self.take(_KV_FMT[t])
            return bool(v) if t == KV_BOOL else v
        if t == KV_STRING:
            return self.string()
        if t == KV_ARRAY:
            et = self.take("<I")
            count = self.take("<Q")
            start = self.o
            if et in _KV_SCALAR:
                size = np.dtype(_KV_SCALAR[et]).itemsize * count
                if self.o + size > self.n:
                    raise GGUFTruncated(f"array of {count} at {start} passes the end")
                self.o += size
            else:
                for _ in range(count):
                    self.value(et)
            return KVArray(self.b, et, count, start, self.o)
        raise GGUFError(f"unknown key/value type {t} at byte {self.o - 4}")


def read_header(buf, partial: bool = False) -> GGUFHeader:
    """Parse the GGUF header in ``buf`` (bytes, mmap or memoryview).

    With ``partial=True`` a buffer that ends inside the tensor list is
    accepted (``truncated`` says where; ``data_offset`` is None), as for a
    partial download; the key/values must be whole either way."""
    if len(buf) < 4 or bytes(buf[:4]) != GGUF_MAGIC:
        raise GGUFError(f"bad magic {bytes(buf[:4])!r}")
    cur = _Cursor(buf, 4)
    version = cur.take("<I")
    if version not in (2, 3):
        raise GGUFError(f"GGUF version {version} is not supported (2 and 3 are)")
    n_tensors = cur.take("<Q")
    n_kv = cur.take("<Q")
    h = GGUFHeader(version=version, n_tensors=n_tensors)
    for _ in range(n_kv):
        key = cur.string()
        t = cur.take("<I")
        h.kv[key] = cur.value(t)
        h.kv_types[key] = t
    align = h.kv.get("general.alignment", GGUF_DEFAULT_ALIGNMENT)
    if h.kv_types.get("general.alignment", KV_U32) != KV_U32 or align <= 0 or align & (align - 1):
        raise GGUFError(f"general.alignment must be a power-of-two u32, got {align!r}")
    h.alignment = align
    try:
        for _ in range(n_tensors):
            name = cur.string()
            nd = cur.take("<I")
            dims = tuple(cur.take("<Q") for _ in range(nd))
            tt = cur.take("<I")
            off = cur.take("<Q")
            h.tensors.append(TensorInfo(name, dims, tt, off))
    except GGUFTruncated as e:
        if not partial:
            raise
        h.truncated = str(e)
        return h
    h.data_offset = (cur.o + align - 1) // align * align
    return h


# ---------------------------------------------------------------- the check
def check_geometry(h: GGUFHeader):
    """The reference tool's verdict on a parsed header.

    Returns ``(fails, report)``: the list of failure messages (empty = the
    file matches the engine) and the lines of the printed report.  Decisions
    follow tools/check_gguf.py:123-173: a key passes when it is stored as
    u32, i32 or string with the expected value; tensors are grouped by
    (layer-generic name, dims, type) and a group of an expected name passes
    when its ne0, ne1 (where fixed), type and, for the counted groups, its
    number of layers match; names matching nextn/mtp/draft/eagle fail the
    file (the engine has no MTP layer)."""
    fails, rep = [], []
    rep.append("metadata keys:")
    for k, want in EXPECT_KV.items():
        got = h.kv.get(k) if h.kv_types.get(k) in _CHECKED_KV_TYPES else None
        ok = got == want
        rep.append(f"  [{'pass' if ok else 'FAIL'}] key {k}: found {got!r}, engine needs {want!r}")
        if not ok:
            fails.append(f"metadata key {k} is {got!r}; the engine is built for {want!r}")

    groups: dict = {}
    mtp = []
    for t in h.tensors:
        if _MTP_RE.search(t.name):
            mtp.append(t.name)
        key = (t.generic_name, t.dims, t.type)
        groups[key] = groups.get(key, 0) + 1
    if h.truncated:
        rep.append(f"  note: only part of the header was readable ({h.truncated}); "
                   "tensors past that point were not checked")

    rep.append("tensor groups (name pattern, shape, type, layers):")
    for (g, dims, tt), cnt in sorted(groups.items()):
        exp = EXPECT_TENSORS.get(g)
        if exp is None:
            continue
        n_in, n_out, etype = exp
        want_count = TENSOR_COUNT.get(g)
        ok = (len(dims) >= 1 and dims[0] == n_in
              and (n_out is None or (len(dims) >= 2 and dims[1] == n_out))
              and tt == etype and (want_count is None or cnt == want_count))
        rep.append(f"  [{'pass' if ok else 'FAIL'}] {g}: shape {list(dims)}, type {tt}, {cnt} of them")
        if not ok:
            need_shape = f"[{n_in}, {n_out}]" if n_out is not None else f"[{n_in}, *]"
            need_count = f", {want_count} of them" if want_count is not None else ""
            fails.append(f"tensor group {g} is shape {list(dims)}, type {tt}, {cnt} of them; "
                         f"the engine needs shape {need_shape}, type {etype}{need_count}")

    if mtp:
        rep.append(f"multi-token-prediction tensors present: {len(mtp)}")
        rep.extend(f"  for instance {n}" for n in mtp[:6])
        fails.append(f"{len(mtp)} multi-token-prediction (nextn) tensors found: this engine runs "
                     "the trunk only, with no draft layer, no batched verification and no second "
                     "KV stream, so a model that needs them cannot run here (its trunk tensors "
                     "are otherwise usable)")
    else:
        rep.append("multi-token-prediction tensors: none, the file is trunk-only as the engine expects")
    return fails, rep


def check_loadable(h: GGUFHeader, file_size: int, layout: str = "native", names=None):
    """What the loader needs beyond the geometry check: for every selected
    PQ2_0 tensor, 2-D with ne0 a positive multiple of 128 (1024 for the
    repack layout, whose kernel works on 8-block groups), data starting on
    the file's alignment and ending inside the file.  Returns the list of
    problems (empty = loadable)."""
    if h.data_offset is None:
        return [f"tensor list incomplete: {h.truncated}"]
    probs = []
    for t in _select(h, names):
        if t.type != GGML_TYPE_PQ2_0:
            probs.append(f"{t.name}: type {t.type} is not PQ2_0")
            continue
        if len(t.dims) != 2 and not (len(t.dims) > 2 and all(d == 1 for d in t.dims[2:])):
            probs.append(f"{t.name}: dims {list(t.dims)} are not 2-D")
            continue
        n_in, n_out = t.dims[0], t.dims[1]
        step = 1024 if layout == "repack" else 128
        if n_in <= 0 or n_out <= 0 or n_in % step:
            probs.append(f"{t.name}: n_in {n_in} must be a positive multiple of {step}")
            continue
        if t.offset % h.alignment:
            probs.append(f"{t.name}: offset {t.offset} is not {h.alignment}-byte aligned")
        end = h.data_offset + t.offset + t.nbytes
        if end > file_size:
            probs.append(f"{t.name}: data ends at byte {end}, the file at {file_size}")
    return probs


def _select(h: GGUFHeader, names):
    if names is None:
        return [t for t in h.tensors if t.type == GGML_TYPE_PQ2_0]
    want = list(names)
    by = {t.name: t for t in h.tensors}
    missing = [n for n in want if n not in by]
    if missing:
        raise KeyError(f"tensors not in the file: {missing}")
    return [by[n] for n in want]


# ---------------------------------------------------------------- the loader
@dataclass(frozen=True)
class PQ2Tensor:
    """One PQ2_0 weight matrix resident in the arena."""
    name: str
    n_in: int
    n_out: int
    layout: str          # "native" (34-byte blocks, rows contiguous) or "repack"
    arena_offset: int
    nbytes: int
    data: object         # torch uint8 view of the arena, nbytes long


@dataclass
class PQ2Weights:
    arena: object                               # one torch uint8 device tensor
    tensors: dict = field(default_factory=dict)  # name -> PQ2Tensor
    layout: str = "native"
    bytes_read: int = 0

    def __getitem__(self, name: str) -> PQ2Tensor:
        return self.tensors[name]

    def __contains__(self, name: str) -> bool:
        return name in self.tensors

    def __len__(self) -> int:
        return len(self.tensors)


def plan_arena(tensors):
    """Slot of each tensor in the arena: 256-byte aligned offsets in file
    order.  Returns (offsets, total bytes)."""
    offs, pos = [], 0
    for t in tensors:
        offs.append(pos)
        pos += (t.nbytes + ARENA_ALIGN - 1) // ARENA_ALIGN * ARENA_ALIGN
    return offs, pos


def load_pq2(path: str, device="cuda", layout: str = "native", names=None,
             staging_bytes: int = 64 << 20, check: bool = False) -> PQ2Weights:
    """Load the PQ2_0 tensors of a GGUF file into device memory.

    ``layout`` "native" keeps the file's bytes (the layout bonsai_p40_gemv,
    _gemm and the grouped GEMVs read); "repack" converts each tensor with
    bonsai_p40_repack for bonsai_p40_gemv_repack.  ``names`` selects tensors
    (default: every PQ2_0 tensor).  ``check=True`` first applies the
    geometry check of the shipped model and raises on any failure.  The file
    is read through mmap in ``staging_bytes`` pieces, alternating between
    two pinned host buffers so reading the file overlaps the copy to HBM."""
    import torch

    if layout not in ("native", "repack"):
        raise ValueError(f"layout must be 'native' or 'repack', got {layout!r}")
    if staging_bytes <= 0 or staging_bytes % ARENA_ALIGN:
        raise ValueError(f"staging_bytes must be a positive multiple of {ARENA_ALIGN}")
    if layout == "repack":
        import bonsai_p40 as B
        B.lib()                                    # fail before any copy if the library is missing
    size = os.path.getsize(path)
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
    try:
        h = read_header(mm)
        if check:
            fails, _ = check_geometry(h)
            if fails:
                raise GGUFError("geometry check failed:\n  " + "\n  ".join(fails))
        probs = check_loadable(h, size, layout, names)
        if probs:
            raise GGUFError("not loadable:\n  " + "\n  ".join(probs))
        sel = _select(h, names)
        offs, total = plan_arena(sel)
        dev = torch.device(device)
        arena = torch.empty(max(total, 1), dtype=torch.uint8, device=dev)
        out = PQ2Weights(arena=arena, layout=layout)
        tmp = None
        if layout == "repack" and sel:
            tmp = torch.empty(max(t.nbytes for t in sel), dtype=torch.uint8, device=dev)
        stage = [torch.empty(staging_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        stage_np = [s.numpy() for s in stage]
        done = [None, None]                       # event after the last copy out of each buffer
        copy_stream = torch.cuda.Stream(dev)       # default priority
        src = np.frombuffer(mm, dtype=np.uint8) if size else np.empty(0, np.uint8)
        k = 0
        with torch.cuda.stream(copy_stream):
            for t, off in zip(sel, offs):
                n = t.nbytes
                base = h.data_offset + t.offset
                dst = arena[off:off + n] if layout == "native" else tmp[:n]
                for p in range(0, n, staging_bytes):
                    m = min(staging_bytes, n - p)
                    i = k & 1
                    if done[i] is not None:
                        done[i].synchronize()      # the copy out of this buffer has finished
                    stage_np[i][:m] = src[base + p:base + p + m]
                    dst[p:p + m].copy_(stage[i][:m], non_blocking=True)
                    ev = torch.cuda.Event()
                    ev.record(copy_stream)
                    done[i] = ev
                    k += 1
                if layout == "repack":
                    B.repack(tmp, arena[off:off + n], t.dims[1], t.dims[0], stream=copy_stream)
                out.tensors[t.name] = PQ2Tensor(t.name, t.dims[0], t.dims[1], layout, off, n,
                                                arena[off:off + n])
                out.bytes_read += n
        copy_stream.synchronize()
        del src
        return out
    finally:
        _close(mm)


def _close(mm) -> None:
    if isinstance(mm, mmap.mmap):
        try:
            mm.close()
        except BufferError:        # a view is still alive (an exception unwinding): leave it to gc
            pass


def load_tensor(path: str, name: str, device="cuda"):
    """One F32/F16/BF16 tensor (norm weights and the like) as a torch tensor
    of shape dims reversed (ne1, ne0)."""
    import torch

    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    try:
        h = read_header(mm)
        t = h.tensor(name)
        dt = {GGML_TYPE_F32: torch.float32, GGML_TYPE_F16: torch.float16,
              GGML_TYPE_BF16: torch.bfloat16}.get(t.type)
        if dt is None:
            raise GGUFError(f"{name}: type {t.type} is not f32/f16/bf16")
        start = h.data_offset + t.offset
        if start + t.nbytes > len(mm):
            raise GGUFError(f"{name}: data ends past the end of the file")
        raw = torch.frombuffer(bytearray(mm[start:start + t.nbytes]), dtype=dt)
        return raw.reshape(tuple(reversed(t.dims))).to(device)
    finally:
        _close(mm)


# ---------------------------------------------------------------- the tool
def main(argv=None) -> int:
    """``gguf_pq2.py [--header] FILE``: the geometry report of a GGUF file
    (``--header``: a file holding only the first bytes of one)."""
    args = list(sys.argv[1:] if argv is None else argv)
    if not args or args[-1].startswith("-"):
        print(main.__doc__)
        return 2
    path = args[-1]
    with open(path, "rb") as f:
        size = os.fstat(f.fileno()).st_size
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
    try:
        try:
            h = read_header(buf, partial=True)
        except GGUFError as e:
            print(f"not usable by this engine: 1 problem\n  * {e}")
            return 1
        print(f"{path}: GGUF version {h.version}, {h.n_tensors} tensors, {len(h.kv)} metadata keys")
        fails, rep = check_geometry(h)
        print("\n".join(rep))
        print()
        if fails:
            print(f"not usable by this engine: {len(fails)} problem{'s' if len(fails) > 1 else ''}")
            for m in fails:
                print("  *", m)
            return 1
        print("usable: every key and tensor group matches the engine's geometry")
        return 0
    finally:
        _close(buf)


if __name__ == "__main__":
    sys.exit(main())
