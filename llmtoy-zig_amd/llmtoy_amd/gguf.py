"""GGUF v1-v3 reader (and a writer for fixtures) feeding real tensors to the
decode path.

The reader follows llmtoy-zig's parser:

  MAGIC, ALIGNMENT, MetaValueType, GgmlType ids   gguf/types.zig:3-53
  Array, MetaValue                                gguf/types.zig:86-122
  TensorInfo.n_elements / byteSize                gguf/types.zig:125-173
  GgufData.meta* lookups                          gguf/reader.zig:7-53
  parseBytes, readMetaValue                       gguf/reader.zig:56-100, 216-235
  GgufReader (map + parse, tensorBytes)           gguf/reader.zig:104-171
  rawMatrix / rawMatrix3D                         model/loader.zig:190-204,
                                                  gemma4/loader.zig:275-292
  MoE layer tensors and config keys               gemma4/loader.zig:27-83, 152-163

Little-endian fields; v1 counts are u32, v2/v3 counts u64; tensor data
starts at the end of the header rounded up to 32 bytes (general.alignment is
not consulted, as in the reference).  Unlike the reference, every read is
bounds-checked: a header or tensor running past the data raises
GgufError("Truncated") instead of reading past the mapping.

The reference has no writer; GgufWriter exists so tests and fixtures can
make files in the layout the reader expects.
"""
from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field
from typing import Any

import numpy as np

from . import ggml

MAGIC = 0x46554747  # "GGUF" little-endian
ALIGNMENT = 32

# MetaValueType (gguf/types.zig:6-20)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# GgmlType id -> (bytes per block, elements per block), gguf/types.zig:138-172.
# Ids without an entry (f64, unknown) have byteSize 0 there.
BLOCK = {
    0: (4, 1), 1: (2, 1), 30: (2, 1), 24: (1, 1), 25: (2, 1), 26: (4, 1), 27: (8, 1),
    2: (18, 32), 3: (20, 32), 6: (22, 32), 7: (24, 32), 8: (34, 32), 9: (40, 32),
    10: (84, 256), 11: (110, 256), 12: (144, 256), 13: (176, 256), 14: (210, 256), 15: (292, 256),
    16: (66, 256), 17: (74, 256), 22: (82, 256), 18: (98, 256), 21: (110, 256), 20: (18, 32),
    23: (136, 256), 19: (50, 256), 29: (56, 256),
}


class GgufError(ValueError):
    """kind: InvalidMagic, UnsupportedVersion, EmptyFile (the reference's
    errors), MissingTensor, MissingMetadata (its loader's LoadError),
    Truncated, BadValueType."""

    def __init__(self, kind: str, msg: str):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind


@dataclass
class Array:
    """An array value: elem_type and the decoded elements (nested arrays are Array)."""
    elem_type: int
    values: list


@dataclass
class TensorInfo:
    name: str
    dims: tuple
    type: int
    offset: int

    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def byte_size(self) -> int:
        """(n / block elements) * block bytes, integer division as in the reference."""
        bb, be = BLOCK.get(self.type, (0, 0))
        return (self.n_elements() // be) * bb if be else 0


@dataclass
class GgufData:
    version: int
    metadata: dict = field(default_factory=dict)  # key -> (MetaValueType, value)
    tensors: list = field(default_factory=list)
    data_offset: int = 0

    def _typed(self, key, *types):
        v = self.metadata.get(key)
        return v[1] if v is not None and v[0] in types else None

    # Each lookup returns None when the key is missing or holds another type.
    def meta_string(self, key):
        return self._typed(key, STRING)

    def meta_u32(self, key):
        return self._typed(key, UINT32)

    def meta_u64(self, key):  # uint32 or uint64 (reader.zig:44-51)
        return self._typed(key, UINT32, UINT64)

    def meta_array(self, key):
        return self._typed(key, ARRAY)

    def meta_bool(self, key):
        return self._typed(key, BOOL)

    def meta_f32(self, key):
        return self._typed(key, FLOAT32)

    def find(self, name):
        for t in self.tensors:
            if t.name == name:
                return t
        return None


class _Cursor:
    def __init__(self, buf):
        self.b = memoryview(buf).cast("B")
        self.pos = 0

    def need(self, k):
        if k > len(self.b) - self.pos:
            raise GgufError("Truncated", "header runs past the end of the data")

    def scalar(self, fmt):
        n = struct.calcsize(fmt)
        self.need(n)
        v = struct.unpack_from(fmt, self.b, self.pos)[0]
        self.pos += n
        return v

    def string(self):
        n = self.scalar("<Q")
        self.need(n)
        s = bytes(self.b[self.pos:self.pos + n]).decode("utf-8", errors="surrogateescape")
        self.pos += n
        return s

    def value(self, t, depth=0):
        if t in _SCALAR:
            return self.scalar(_SCALAR[t])
        if t == BOOL:
            return self.scalar("<B") != 0
        if t == STRING:
            return self.string()
        if t == ARRAY:
            if depth > 8:
                raise GgufError("BadValueType", "arrays nested too deeply")
            et = self.scalar("<I")
            n = self.scalar("<Q")
            self.need(n)  # every element is at least one byte
            return Array(et, [self.value(et, depth + 1) for _ in range(n)])
        raise GgufError("BadValueType", f"unknown metadata value type {t}")


def parse_bytes(buf) -> GgufData:
    """Parse a GGUF header from bytes (gguf/reader.zig:56-100)."""
    c = _Cursor(buf)
    if c.scalar("<I") != MAGIC:
        raise GgufError("InvalidMagic", "not a GGUF file")
    version = c.scalar("<I")
    if version < 1 or version > 3:
        raise GgufError("UnsupportedVersion", f"version {version}")
    cnt = "<I" if version == 1 else "<Q"
    n_tensors, n_kv = c.scalar(cnt), c.scalar(cnt)
    g = GgufData(version)
    for _ in range(n_kv):
        key = c.string()
        t = c.scalar("<I")
        g.metadata[key] = (t, c.value(t))  # a repeated key keeps the last value
    c.need(n_tensors)
    for _ in range(n_tensors):
        name = c.string()
        nd = c.scalar("<I")
        c.need(8 * nd)
        dims = tuple(c.scalar("<Q") for _ in range(nd))
        g.tensors.append(TensorInfo(name, dims, c.scalar("<I"), c.scalar("<Q")))
    g.data_offset = (c.pos + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT
    return g


@dataclass
class RawMatrix:
    """model/model_weights.zig:17-22: rows x cols of one GGUF type; data is a
    uint8 [rows, row_bytes] view of the mapped file."""
    data: np.ndarray
    type: int
    rows: int
    cols: int


class GgufReader:
    """A GGUF file mapped read-only and parsed (gguf/reader.zig:104-171).
    Tensor views stay valid while the reader is referenced."""

    def __init__(self, path: str):
        if os.path.getsize(path) == 0:
            raise GgufError("EmptyFile", path)
        self.map = np.memmap(path, dtype=np.uint8, mode="r")
        self.data = parse_bytes(self.map)

    def tensor(self, name: str) -> TensorInfo:
        t = self.data.find(name)
        if t is None:
            raise GgufError("MissingTensor", name)
        return t

    def tensor_bytes(self, info: TensorInfo) -> np.ndarray:
        """Exactly byte_size() bytes of the tensor (tensorBytes)."""
        start, n = self.data.data_offset + info.offset, info.byte_size()
        if start + n > self.map.size:
            raise GgufError("Truncated", f"tensor {info.name} runs past the end of the file")
        return self.map[start:start + n]

    def raw_matrix(self, name: str, rows: int, cols: int) -> RawMatrix:
        """model/loader.zig:190-204, shape from the model config.  The tensor
        must hold rows whole rows (the device upload reads rows * row_bytes)."""
        t = self.tensor(name)
        raw = self.tensor_bytes(t)
        bb, be = BLOCK.get(t.type, (0, 0))
        if not be or cols % be or rows * (cols // be) * bb > raw.size:
            raise GgufError("Truncated", f"tensor {name} does not hold {rows} rows of {cols}")
        rb = (cols // be) * bb
        return RawMatrix(raw[:rows * rb].reshape(rows, rb), t.type, rows, cols)

    def raw_matrix_3d(self, name: str, n_experts: int, rows_per_expert: int, cols: int) -> RawMatrix:
        """gemma4/loader.zig:275-292: [cols, rows_per_expert, n_experts] as one
        matrix of n_experts * rows_per_expert rows."""
        return self.raw_matrix(name, n_experts * rows_per_expert, cols)

    def meta_string(self, key):
        return self.data.meta_string(key)

    def meta_u32(self, key):
        return self.data.meta_u32(key)

    def meta_u64(self, key):
        return self.data.meta_u64(key)

    def meta_array(self, key):
        return self.data.meta_array(key)

    def meta_bool(self, key):
        return self.data.meta_bool(key)

    def meta_f32(self, key):
        return self.data.meta_f32(key)


# ---------------------------------------------------------------- MoE layer
@dataclass
class MoEConfig:
    arch: str
    d_model: int
    n_experts: int
    n_experts_used: int
    d_expert: int


def moe_config(r: GgufReader) -> MoEConfig:
    """The MoE shape keys, read as gemma4/loader.zig:27-75 reads them
    ({arch}.embedding_length, .expert_count, .expert_used_count (default 8),
    .expert_feed_forward_length)."""
    arch = r.meta_string("general.architecture")
    if arch is None:
        raise GgufError("MissingMetadata", "general.architecture")

    def need(k):
        v = r.meta_u64(f"{arch}.{k}")
        if v is None:
            raise GgufError("MissingMetadata", f"{arch}.{k}")
        return int(v)

    used = r.meta_u64(f"{arch}.expert_used_count")
    return MoEConfig(arch, need("embedding_length"), need("expert_count"), 8 if used is None else int(used),
                     need("expert_feed_forward_length"))


@dataclass
class MoELayer:
    """One layer's MoE tensors in the shapes the device path takes (the same
    fields as synth.MoEWeights, so lib.upload_moe uploads either)."""
    d_model: int
    n_experts: int
    d_expert: int
    down_cols: int
    router: np.ndarray
    router_type: int
    gate_up: np.ndarray
    down: np.ndarray
    gate_up_type: int
    down_type: int
    extra: dict = field(default_factory=dict)


def load_moe_layer(r: GgufReader, layer: int, cfg: MoEConfig | None = None) -> MoELayer:
    """blk.{layer}.ffn_gate_inp.weight (router [E, d]), ffn_gate_up_exps.weight
    ([d, 2F, E]: per expert F gate rows then F up rows) and
    ffn_down_exps.weight ([F, d, E]), as gemma4/loader.zig:152-163.  A file
    with separate ffn_gate_exps / ffn_up_exps tensors ([d, F, E] each, the
    llama.cpp Qwen3-MoE naming) is accepted too: its gate and up rows are
    interleaved per expert into one host copy.  The optional per-expert
    ffn_down_exps.scale and router-input ffn_gate_inp.scale (F32) land in
    extra; this function applies neither."""
    cfg = cfg or moe_config(r)
    d, E, F = cfg.d_model, cfg.n_experts, cfg.d_expert
    p = f"blk.{layer}."
    router = r.raw_matrix(p + "ffn_gate_inp.weight", E, d)
    if r.data.find(p + "ffn_gate_up_exps.weight") is not None:
        gu = r.raw_matrix_3d(p + "ffn_gate_up_exps.weight", E, 2 * F, d)
        gate_up, gu_type = gu.data, gu.type
    else:
        g = r.raw_matrix_3d(p + "ffn_gate_exps.weight", E, F, d)
        u = r.raw_matrix_3d(p + "ffn_up_exps.weight", E, F, d)
        if g.type != u.type:
            raise GgufError("BadValueType", "gate and up experts have different types")
        rb = g.data.shape[1]
        gate_up = np.empty((E, 2, F, rb), dtype=np.uint8)
        gate_up[:, 0] = g.data.reshape(E, F, rb)
        gate_up[:, 1] = u.data.reshape(E, F, rb)
        gate_up, gu_type = gate_up.reshape(E * 2 * F, rb), g.type
    dn_info = r.tensor(p + "ffn_down_exps.weight")
    down_cols = dn_info.dims[0] if dn_info.dims else F
    dn = r.raw_matrix_3d(p + "ffn_down_exps.weight", E, d, down_cols)
    extra = {}
    for key, n in (("ffn_down_exps.scale", E), ("ffn_gate_inp.scale", d)):
        t = r.data.find(p + key)
        if t is not None:
            if t.type != ggml.F32 or t.n_elements() != n:
                raise GgufError("BadValueType", f"{p + key} is not F32[{n}]")
            extra[key] = r.tensor_bytes(t).view(np.float32)
    router_data = router.data.view(np.float32) if router.type == ggml.F32 else router.data
    return MoELayer(d, E, F, down_cols, router_data, router.type, gate_up, dn.data, gu_type, dn.type, extra)


def _load_vec(r: GgufReader, name: str, n: int) -> np.ndarray:
    """gemma4/loader.zig:182-199 loadNorm: an F32 or F16 vector of n values."""
    t = r.tensor(name)
    if t.n_elements() != n:
        raise GgufError("BadValueType", f"{name} has {t.n_elements()} values, expected {n}")
    raw = r.tensor_bytes(t)
    if t.type == ggml.F32:
        return raw.view(np.float32).copy()
    if t.type == ggml.F16:
        return raw.view(np.float16).astype(np.float32)
    raise GgufError("BadValueType", f"{name}: type {t.type} (norms are F32 or F16)")


def load_gemma4_norms(r: GgufReader, layer: int, cfg: MoEConfig | None = None) -> tuple:
    """The vectors of a Gemma4 MoE block (gemma4/loader.zig:121-163):
    (norms dict for lt gemma4_moe_block, layer_output_scale).  A missing
    layer_output_scale is 1, as loadScalar returns (201-214)."""
    cfg = cfg or moe_config(r)
    d, E = cfg.d_model, cfg.n_experts
    p = f"blk.{layer}."
    norms = {"pre_ffw_norm_2": _load_vec(r, p + "pre_ffw_norm_2.weight", d),
             "router_scale": _load_vec(r, p + "ffn_gate_inp.scale", d),
             "down_exps_scale": _load_vec(r, p + "ffn_down_exps.scale", E),
             "post_ffw_norm_2": _load_vec(r, p + "post_ffw_norm_2.weight", d),
             "post_ffw_norm": _load_vec(r, p + "post_ffw_norm.weight", d)}
    t = r.data.find(p + "layer_output_scale.weight")
    los = 1.0 if t is None or t.type not in (ggml.F32, ggml.F16) else float(_load_vec(r, t.name, 1)[0])
    return norms, los


# ---------------------------------------------------------------- writer
class GgufWriter:
    """Builds GGUF files: header, metadata, tensor infos, then each tensor's
    bytes at a 32-byte aligned offset from the data start."""

    def __init__(self, version: int = 3):
        self.version = version
        self.kv: list[tuple[str, int, Any]] = []
        self.tensors: list[tuple[str, tuple, int, bytes]] = []

    def add(self, key: str, vtype: int, value):
        """value: a Python scalar/str/bool, or Array(elem_type, values) for ARRAY."""
        self.kv.append((key, vtype, value))
        return self

    def add_tensor(self, name: str, dims, ggml_type: int, data):
        """dims in GGUF order (innermost first: [cols, rows, experts])."""
        b = np.ascontiguousarray(data).view(np.uint8).tobytes() if isinstance(data, np.ndarray) else bytes(data)
        info = TensorInfo(name, tuple(int(x) for x in dims), ggml_type, 0)
        if len(b) != info.byte_size():
            raise ValueError(f"{name}: {len(b)} bytes for a tensor of {info.byte_size()}")
        self.tensors.append((name, info.dims, ggml_type, b))
        return self

    @staticmethod
    def _str(s: str) -> bytes:
        e = s.encode("utf-8", errors="surrogateescape")
        return struct.pack("<Q", len(e)) + e

    def _value(self, t, v) -> bytes:
        if t in _SCALAR:
            return struct.pack(_SCALAR[t], v)
        if t == BOOL:
            return struct.pack("<B", 1 if v else 0)
        if t == STRING:
            return self._str(v)
        if t == ARRAY:
            return struct.pack("<IQ", v.elem_type, len(v.values)) + b"".join(
                self._value(v.elem_type, x) for x in v.values)
        raise ValueError(f"unknown value type {t}")

    def to_bytes(self) -> bytes:
        cnt = "<I" if self.version == 1 else "<Q"
        out = [struct.pack("<II", MAGIC, self.version), struct.pack(cnt, len(self.tensors)),
               struct.pack(cnt, len(self.kv))]
        for key, t, v in self.kv:
            out += [self._str(key), struct.pack("<I", t), self._value(t, v)]
        off, blobs = 0, []
        for name, dims, t, b in self.tensors:
            out += [self._str(name), struct.pack("<I", len(dims)), struct.pack(f"<{len(dims)}Q", *dims),
                    struct.pack("<IQ", t, off)]
            pad = (-len(b)) % ALIGNMENT
            blobs += [b, bytes(pad)]
            off += len(b) + pad
        head = b"".join(out)
        head += bytes((-len(head)) % ALIGNMENT)
        return head + b"".join(blobs)

    def write(self, path: str):
        with open(path, "wb") as f:
            f.write(self.to_bytes())
        return path


def moe_layer_writer(w, layer: int = 0, arch: str = "qwen3moe", k: int = 8, split: bool = False,
                     version: int = 3, extra: dict | None = None) -> GgufWriter:
    """A writer holding synth.MoEWeights as one layer, in the tensor layout
    load_moe_layer reads (split=True: separate gate and up experts).
    extra: name suffix -> F32 array (e.g. "ffn_down_exps.scale")."""
    E, F, d, dc = w.n_experts, w.d_expert, w.d_model, w.down_cols
    wr = GgufWriter(version)
    wr.add("general.architecture", STRING, arch)
    wr.add(f"{arch}.embedding_length", UINT32, d)
    wr.add(f"{arch}.expert_count", UINT32, E)
    wr.add(f"{arch}.expert_used_count", UINT32, k)
    wr.add(f"{arch}.expert_feed_forward_length", UINT32, F)
    p = f"blk.{layer}."
    wr.add_tensor(p + "ffn_gate_inp.weight", (d, E), w.router_type, w.router)
    gut, dnt = getattr(w, "gate_up_type", ggml.Q4_K), getattr(w, "down_type", ggml.Q4_K)
    if split:
        gu = w.gate_up.reshape(E, 2, F, -1)
        wr.add_tensor(p + "ffn_gate_exps.weight", (d, F, E), gut, gu[:, 0])
        wr.add_tensor(p + "ffn_up_exps.weight", (d, F, E), gut, gu[:, 1])
    else:
        wr.add_tensor(p + "ffn_gate_up_exps.weight", (d, 2 * F, E), gut, w.gate_up)
    wr.add_tensor(p + "ffn_down_exps.weight", (dc, d, E), dnt, w.down)
    for key, arr in (extra or {}).items():
        arr = np.asarray(arr, dtype=np.float32)
        wr.add_tensor(p + key, (arr.size,), ggml.F32, arr)
    return wr


def write_moe_layer(path: str, w, **kw) -> str:
    """moe_layer_writer(w, **kw) written to path."""
    return moe_layer_writer(w, **kw).write(path)
