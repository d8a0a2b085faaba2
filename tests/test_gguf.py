"""GGUF reader (llmtoy_amd/gguf.py, host/gguf_reader.hpp): parse tests pinned
by hand-packed bytes (the reference's own parseBytes test, gguf/reader.zig:
247-297, and one value of every metadata type), block-size closed forms,
error cases, Python/C++ agreement on written files, and -- on the GPU --
MoE layers and matvec weights read from a GGUF file run through the device
path and checked against the oracle on the same bytes."""
import os
import struct
import subprocess

import numpy as np
import pytest

import llmtoy_amd as lt
from llmtoy_amd import ggml, gguf, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# LT_TEST_GGUF_BIN: another build of the same test (the sanitizer build)
CPP = os.environ.get("LT_TEST_GGUF_BIN") or os.path.join(ROOT, "tests", "cpp", "build", "test_gguf")


def s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def reference_kat():
    """gguf/reader.zig:247-297, restated: header end and the padded file."""
    b = struct.pack("<IIQQ", gguf.MAGIC, 3, 1, 2)
    b += s("general.architecture") + struct.pack("<I", 8) + s("test_arch")
    b += s("test.context_length") + struct.pack("<II", 4, 256)
    b += s("weight") + struct.pack("<IQQIQ", 2, 4, 4, 0, 0)
    end = len(b)
    return end, b + bytes((-end) % 32) + bytes(64)


def test_reference_kat():
    end, b = reference_kat()
    g = gguf.parse_bytes(b)
    assert g.version == 3 and len(g.metadata) == 2 and len(g.tensors) == 1
    assert g.meta_string("general.architecture") == "test_arch"
    assert g.meta_u32("test.context_length") == 256
    t = g.tensors[0]
    assert t.name == "weight" and t.n_elements() == 16 and t.type == ggml.F32 and t.byte_size() == 64
    # 24 header + 49 + 35 metadata + 46 tensor info = 154, aligned to 32
    assert end == 154 and g.data_offset == 160


def test_every_header_prefix_is_truncated():
    end, b = reference_kat()
    for n in range(end):
        with pytest.raises(gguf.GgufError) as e:
            gguf.parse_bytes(b[:n])
        assert e.value.kind == "Truncated", n
    assert gguf.parse_bytes(b[:end]).data_offset == 160


@pytest.mark.parametrize("version", [0, 4, 0xFFFFFFFF])
def test_unsupported_version(version):
    _, b = reference_kat()
    with pytest.raises(gguf.GgufError) as e:
        gguf.parse_bytes(b[:4] + struct.pack("<I", version) + b[8:])
    assert e.value.kind == "UnsupportedVersion"


def test_invalid_magic():
    _, b = reference_kat()
    with pytest.raises(gguf.GgufError) as e:
        gguf.parse_bytes(b"GGUG" + b[4:])
    assert e.value.kind == "InvalidMagic"


def test_v1_counts_are_u32():
    b = struct.pack("<IIII", gguf.MAGIC, 1, 1, 1) + s("k") + struct.pack("<IQ", 10, 0x0123456789ABCDEF)
    b += s("t") + struct.pack("<IQIQ", 1, 32, 8, 0)
    end = len(b)
    g = gguf.parse_bytes(b + bytes((-end) % 32) + bytes(34))
    assert g.version == 1 and g.meta_u64("k") == 0x0123456789ABCDEF
    assert g.tensors[0].byte_size() == 34 and g.data_offset == (end + 31) // 32 * 32


def test_every_value_type():
    kv = [("u8", 0, "<B", 200), ("i8", 1, "<b", -100), ("u16", 2, "<H", 60000), ("i16", 3, "<h", -30000),
          ("u32", 4, "<I", 4000000000), ("i32", 5, "<i", -2000000000), ("f32", 6, "<f", -1.5),
          ("u64", 10, "<Q", 18000000000000000000), ("i64", 11, "<q", -9000000000000000000), ("f64", 12, "<d", 0.1)]
    b = b"".join(s(k) + struct.pack("<I", t) + struct.pack(f, v) for k, t, f, v in kv)
    b += s("bool") + struct.pack("<IB", 7, 2)  # any non-zero byte is true
    b += s("str") + struct.pack("<I", 8) + struct.pack("<Q", 6) + "héllo".encode()
    b += s("arr") + struct.pack("<IIQ", 9, 8, 2) + s("a") + s("")
    b += s("nest") + struct.pack("<IIQ", 9, 9, 2) + struct.pack("<IQi", 5, 1, -7) + struct.pack("<IQ", 6, 0)
    g = gguf.parse_bytes(struct.pack("<IIQQ", gguf.MAGIC, 2, 0, 14) + b)
    for k, t, _, v in kv:
        assert g.metadata[k] == (t, v), k
    assert g.meta_bool("bool") is True and g.meta_string("str") == "héllo"
    assert g.meta_array("arr") == gguf.Array(gguf.STRING, ["a", ""])
    assert g.meta_array("nest") == gguf.Array(gguf.ARRAY, [gguf.Array(gguf.INT32, [-7]), gguf.Array(gguf.FLOAT32, [])])
    # typed lookups: None for another type or a missing key; meta_u64 takes uint32 too
    assert g.meta_u32("u64") is None and g.meta_string("u8") is None and g.meta_f32("f64") is None
    assert g.meta_array("missing") is None and g.meta_u64("u32") == 4000000000


def test_bad_value_type_and_oversized_counts():
    with pytest.raises(gguf.GgufError) as e:
        gguf.parse_bytes(struct.pack("<IIQQ", gguf.MAGIC, 3, 0, 1) + s("x") + struct.pack("<II", 13, 0))
    assert e.value.kind == "BadValueType"
    for b in (struct.pack("<IIQQ", gguf.MAGIC, 3, 0, 1) + s("x") + struct.pack("<IIQ", 9, 0, 1 << 60),
              struct.pack("<IIQQ", gguf.MAGIC, 3, 1 << 50, 0)):
        with pytest.raises(gguf.GgufError) as e:
            gguf.parse_bytes(b)
        assert e.value.kind == "Truncated"


# Block bytes from each block layout (d/dmin halves, scale bytes, packed quants).
LAYOUTS = {0: (4, 1), 1: (2, 1), 30: (2, 1), 24: (1, 1), 25: (2, 1), 26: (4, 1), 27: (8, 1),
           2: (2 + 16, 32), 3: (2 + 2 + 16, 32), 6: (2 + 4 + 16, 32), 7: (2 + 2 + 4 + 16, 32), 8: (2 + 32, 32),
           9: (4 + 4 + 32, 32),  # q8_1 as the reference sizes it (f32 d and s)
           10: (16 + 64 + 2 + 2, 256), 11: (32 + 64 + 12 + 2, 256), 12: (2 + 2 + 12 + 128, 256),
           13: (2 + 2 + 12 + 32 + 128, 256), 14: (128 + 64 + 16 + 2, 256), 15: (4 + 256 + 32, 256)}


def test_byte_size_matches_block_layouts():
    for t, (bb, be) in LAYOUTS.items():
        assert gguf.BLOCK[t] == (bb, be), t
        assert gguf.TensorInfo("x", (be * 8, 3), t, 0).byte_size() == 24 * bb
    assert gguf.TensorInfo("x", (5,), 28, 0).byte_size() == 0  # f64: no entry in the reference table
    for t in (ggml.F32, ggml.F16, ggml.Q8_0, ggml.Q4_K, ggml.Q6_K):
        assert gguf.TensorInfo("x", (1024, 5), t, 0).byte_size() == 5 * ggml.row_bytes(t, 1024)


def writer_sample(version):
    w = gguf.GgufWriter(version)
    w.add("general.architecture", gguf.STRING, "qwen3moe")
    for i, (t, v) in enumerate([(gguf.UINT8, 7), (gguf.INT8, -7), (gguf.UINT16, 65535), (gguf.INT16, -1),
                                (gguf.UINT32, 1 << 31), (gguf.INT32, -5), (gguf.FLOAT32, 0.25), (gguf.BOOL, False),
                                (gguf.UINT64, (1 << 64) - 1), (gguf.INT64, -(1 << 63)), (gguf.FLOAT64, -2.5e-300)]):
        w.add(f"k{i}", t, v)
    w.add("tok", gguf.ARRAY, gguf.Array(gguf.STRING, ["<s>", "é", ""]))
    w.add("nested", gguf.ARRAY, gguf.Array(gguf.ARRAY, [gguf.Array(gguf.UINT8, [1, 2]), gguf.Array(gguf.BOOL, [True])]))
    g = synth.stream(99, 0)
    w.add_tensor("a.q4k", (512, 3), ggml.Q4_K, synth.q4k_matrix(g, 3, 512))
    w.add_tensor("b.q8", (64, 5), ggml.Q8_0, synth.q8_0_matrix(g, 5, 64))
    w.add_tensor("c.f32", (7,), ggml.F32, np.arange(7, dtype=np.float32))
    w.add_tensor("d.q6k", (256, 2, 2), ggml.Q6_K, synth.q6k_matrix(g, 4, 256))
    return w


@pytest.mark.parametrize("version", [1, 2, 3])
def test_writer_reader_round_trip(version, tmp_path):
    w = writer_sample(version)
    p = w.write(str(tmp_path / "s.gguf"))
    r = gguf.GgufReader(p)
    assert r.data.version == version and r.data.data_offset % 32 == 0
    assert {k: (t, v) for k, t, v in w.kv} == r.data.metadata
    for (name, dims, t, b), info in zip(w.tensors, r.data.tensors):
        assert (info.name, info.dims, info.type) == (name, dims, t) and info.offset % 32 == 0
        assert r.tensor_bytes(info).tobytes() == b


def canonical_dump(r: gguf.GgufReader) -> str:
    """The C++ test binary's --dump format."""
    def val(t, v):
        if t == gguf.FLOAT32:
            return "f%08x" % struct.unpack("<I", struct.pack("<f", v))[0]
        if t == gguf.FLOAT64:
            return "d%016x" % struct.unpack("<Q", struct.pack("<d", v))[0]
        if t == gguf.BOOL:
            return "true" if v else "false"
        if t == gguf.STRING:
            return "s" + v.encode("utf-8", errors="surrogateescape").hex()
        if t == gguf.ARRAY:
            return "[%d:%s]" % (v.elem_type, ",".join(val(v.elem_type, x) for x in v.values))
        return str(v)

    def fnv1a(b):
        h = 0xCBF29CE484222325
        for c in b:
            h = ((h ^ c) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
        return h

    lines = [f"version {r.data.version}", f"data_offset {r.data.data_offset}"]
    for k in sorted(r.data.metadata, key=lambda k: k.encode()):
        t, v = r.data.metadata[k]
        lines.append(f"kv {k} {t} {val(t, v)}")
    for t in r.data.tensors:
        lines.append("tensor %s %d %d %s %d %d %016x" % (t.name, t.type, t.offset, ",".join(map(str, t.dims)),
                                                          t.n_elements(), t.byte_size(),
                                                          fnv1a(r.tensor_bytes(t).tobytes())))
    return "\n".join(lines) + "\n"


def test_cpp_reader_tests_pass():
    out = subprocess.run([CPP, "--cpu"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0 and "ALL PASSED" in out.stdout, out.stdout + out.stderr
    names = subprocess.run([CPP, "--list"], capture_output=True, text=True, timeout=60).stdout.splitlines()
    assert "parseBytes: synthetic GGUF v3" in names and len(names) == 9


@pytest.mark.parametrize("version", [1, 3])
def test_cpp_and_python_readers_agree(version, tmp_path):
    p = writer_sample(version).write(str(tmp_path / "s.gguf"))
    out = subprocess.run([CPP, "--dump", p], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout == canonical_dump(gguf.GgufReader(p))


def test_reader_errors(tmp_path):
    e = tmp_path / "empty.gguf"
    e.write_bytes(b"")
    with pytest.raises(gguf.GgufError) as x:
        gguf.GgufReader(str(e))
    assert x.value.kind == "EmptyFile"
    full = writer_sample(3).to_bytes()
    p = tmp_path / "cut.gguf"
    p.write_bytes(full[:-40])  # the last tensor loses its tail
    r = gguf.GgufReader(str(p))
    with pytest.raises(gguf.GgufError) as x:
        r.tensor_bytes(r.tensor("d.q6k"))
    assert x.value.kind == "Truncated"
    with pytest.raises(gguf.GgufError) as x:
        r.tensor("nope")
    assert x.value.kind == "MissingTensor"
    with pytest.raises(gguf.GgufError) as x:
        r.raw_matrix_3d("a.q4k", 2, 2, 512)  # 4 rows from a 3-row tensor
    assert x.value.kind == "Truncated"
    m = r.raw_matrix("a.q4k", 3, 512)
    assert m.data.shape == (3, 288) and m.type == ggml.Q4_K


@pytest.mark.parametrize("split", [False, True])
def test_moe_layer_from_gguf_is_the_written_bytes(split, tmp_path):
    w = synth.moe_weights(3, 512, 8, 256)
    scale = np.linspace(0.5, 1.5, 8, dtype=np.float32)
    p = gguf.write_moe_layer(str(tmp_path / "m.gguf"), w, layer=2, k=4, split=split,
                             extra={"ffn_down_exps.scale": scale})
    r = gguf.GgufReader(p)
    cfg = gguf.moe_config(r)
    assert (cfg.d_model, cfg.n_experts, cfg.n_experts_used, cfg.d_expert) == (512, 8, 4, 256)
    L = gguf.load_moe_layer(r, 2)
    assert np.array_equal(L.router, w.router) and np.array_equal(L.gate_up, w.gate_up)
    assert np.array_equal(L.down, w.down) and L.down_cols == w.down_cols
    assert np.array_equal(L.extra["ffn_down_exps.scale"], scale)
    with pytest.raises(gguf.GgufError) as x:
        gguf.load_moe_layer(r, 0)
    assert x.value.kind == "MissingTensor"


def test_moe_config_defaults_and_missing_keys(tmp_path):
    w = gguf.GgufWriter(3).add("general.architecture", gguf.STRING, "a")
    for k, v in (("embedding_length", 512), ("expert_count", 8), ("expert_feed_forward_length", 256)):
        w.add(f"a.{k}", gguf.UINT64, v)
    w.add_tensor("x", (1,), ggml.F32, np.zeros(1, np.float32))
    cfg = gguf.moe_config(gguf.GgufReader(w.write(str(tmp_path / "c.gguf"))))
    assert cfg.n_experts_used == 8  # gemma4/loader.zig:75 default
    w.kv = w.kv[:2]
    with pytest.raises(gguf.GgufError) as x:
        gguf.moe_config(gguf.GgufReader(w.write(str(tmp_path / "d.gguf"))))
    assert x.value.kind == "MissingMetadata"


# ------------------------------------------------------------------ GPU
def write_test_file(path, w, k=8, split=False, scale=None):
    """One MoE layer plus matvec weights and their input vectors (test.*)."""
    g = synth.stream(98, 0)
    x = synth.normal(g, (w.d_model,))
    wr = gguf.moe_layer_writer(w, k=k, split=split, extra={} if scale is None else {"ffn_down_exps.scale": scale})
    wr.add_tensor("test.x", (w.d_model,), ggml.F32, x)
    wr.add_tensor("test.q8_0", (1024, 96), ggml.Q8_0, synth.q8_0_matrix(g, 96, 1024))
    wr.add_tensor("test.q6_k", (1024, 80), ggml.Q6_K, synth.q6k_matrix(g, 80, 1024))
    wr.add_tensor("test.q4_k", (1024, 64), ggml.Q4_K, synth.q4k_matrix(g, 64, 1024))
    for t, name in ((ggml.Q5_0, "q5_0"), (ggml.Q5_1, "q5_1"), (ggml.IQ4_NL, "iq4_nl"), (ggml.Q3_K, "q3_k")):
        wr.add_tensor(f"test.{name}", (1024, 48), t, synth.quant_matrix(g, t, 48, 1024))
    wr.add_tensor("test.v1024", (1024,), ggml.F32, synth.normal(g, (1024,)))
    wr.write(path)
    return x


@pytest.mark.gpu
@pytest.mark.parametrize("split", [False, True])
def test_gpu_moe_layer_from_gguf(ctx, split, tmp_path):
    import pyoracle as orc
    w = synth.moe_weights(3, 1024, 32, 512)
    p = str(tmp_path / "layer.gguf")
    x = write_test_file(p, w, split=split)
    print(f"gguf moe layer split={split} {p}", flush=True)
    r = gguf.GgufReader(p)
    L = gguf.load_moe_layer(r, 0)
    xs = r.tensor_bytes(r.tensor("test.x")).view(np.float32)
    assert np.array_equal(xs, x)
    outs = []
    for src in (L, w):  # weights read from the file vs the in-memory synth weights
        R, GU, DN = lt.upload_moe(ctx, src)
        o = np.zeros(w.d_model, np.float32)
        ids = np.zeros(8, np.uint32)
        ctx.moe_forward(o, xs, R, GU, DN, 8, w.d_expert, out_ids=ids, deterministic=True)
        outs.append((o, ids))
        for t in (R, GU, DN):
            t.free()
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    ref, rids, _, agree = orc.moe_forward(w, x, 8)
    assert agree and np.array_equal(np.sort(outs[0][1]), np.sort(rids))
    err = float(np.linalg.norm(outs[0][0].astype(np.float64) - ref) / np.linalg.norm(ref))
    assert err < 1e-3, err


@pytest.mark.gpu
def test_gpu_matvec_weights_from_gguf(ctx, tmp_path):
    import pyoracle as orc
    w = synth.moe_weights(3, 512, 8, 256)
    p = str(tmp_path / "mv.gguf")
    write_test_file(p, w)
    r = gguf.GgufReader(p)
    v = r.tensor_bytes(r.tensor("test.v1024")).view(np.float32)
    for name in ("test.q8_0", "test.q6_k", "test.q4_k", "test.q5_0", "test.q5_1", "test.iq4_nl", "test.q3_k"):
        info = r.tensor(name)
        m = r.raw_matrix(name, info.dims[1], info.dims[0])
        print(f"gguf matvec {name} {m.rows}x{m.cols}", flush=True)
        t = ctx.upload(m.data, m.type, m.rows, m.cols)
        y = np.zeros(m.rows, np.float32)
        ctx.quant_matvec(y, t, v)
        t.free()
        ref = orc.quant_matvec(np.asarray(m.data), m.type, v, m.rows, m.cols)
        assert float(np.linalg.norm(y.astype(np.float64) - ref) / np.linalg.norm(ref)) < 1e-3, name


@pytest.mark.gpu
@pytest.mark.parametrize("split", [False, True])
def test_gpu_cpp_reader_runs_gguf_layer(split, tmp_path):
    w = synth.moe_weights(3, 1024, 32, 512)
    p = str(tmp_path / "cpp.gguf")
    write_test_file(p, w, split=split, scale=np.linspace(0.25, 2.0, 32, dtype=np.float32))
    print(f"running tests/cpp/build/test_gguf --gpu split={split}", flush=True)
    out = subprocess.run([CPP, "--gpu", p], capture_output=True, text=True, timeout=120)
    print(out.stdout[-3000:])
    assert out.returncode == 0 and "ALL PASSED" in out.stdout, out.stdout + out.stderr


def write_gemma4_layer(path, w, nm, los, version=3):
    """A Gemma4 MoE block's tensors under the loader's names (gemma4/loader.zig:121-163)."""
    wr = gguf.moe_layer_writer(w, arch="gemma4", version=version,
                               extra={"ffn_down_exps.scale": nm["down_exps_scale"],
                                      "ffn_gate_inp.scale": nm["router_scale"]})
    for key in ("pre_ffw_norm_2", "post_ffw_norm_2", "post_ffw_norm"):
        wr.add_tensor(f"blk.0.{key}.weight", (w.d_model,), ggml.F32, nm[key])
    wr.add_tensor("blk.0.layer_output_scale.weight", (1,), ggml.F32, np.array([los], np.float32))
    return wr.write(path)


def test_gemma4_norms_from_gguf(tmp_path):
    w = synth.moe_weights(46, 512, 8, 256, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K, down_type=ggml.IQ4_NL)
    nm = synth.gemma4_norms(46, 512, 8)
    r = gguf.GgufReader(write_gemma4_layer(str(tmp_path / "g4.gguf"), w, nm, 0.625))
    got, los = gguf.load_gemma4_norms(r, 0)
    assert los == 0.625 and all(np.array_equal(got[k], nm[k]) for k in nm)
    L = gguf.load_moe_layer(r, 0)
    assert (L.gate_up_type, L.down_type, L.router_type) == (ggml.Q3_K, ggml.IQ4_NL, ggml.Q8_0)
    assert np.array_equal(L.gate_up, w.gate_up) and np.array_equal(L.down, w.down)


@pytest.mark.gpu
def test_gpu_cpp_reader_runs_gemma4_block(tmp_path):
    # the C++ reader and host layer: gemma4Norms + GpuWeights::runMoeBlock from a file
    w = synth.moe_weights(49, 2816, 16, 704, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                          down_type=ggml.IQ4_NL)
    nm = synth.gemma4_norms(49, 2816, 16)
    wr = gguf.moe_layer_writer(w, arch="gemma4", extra={"ffn_down_exps.scale": nm["down_exps_scale"],
                                                         "ffn_gate_inp.scale": nm["router_scale"]})
    for key in ("pre_ffw_norm_2", "post_ffw_norm_2", "post_ffw_norm"):
        wr.add_tensor(f"blk.0.{key}.weight", (2816,), ggml.F16 if key == "post_ffw_norm" else ggml.F32,
                      nm[key].astype(np.float16) if key == "post_ffw_norm" else nm[key])
    wr.add_tensor("blk.0.layer_output_scale.weight", (1,), ggml.F32, np.array([0.75], np.float32))
    wr.add_tensor("test.x", (2816,), ggml.F32, synth.normal(synth.stream(49, 1), (2816,)))
    wr.add_tensor("test.dense", (2816,), ggml.F32, synth.normal(synth.stream(49, 2), (2816,)))
    p = wr.write(str(tmp_path / "g4cpp.gguf"))
    print("running tests/cpp/build/test_gguf --gpu on a Gemma4 block file", flush=True)
    out = subprocess.run([CPP, "--gpu", p], capture_output=True, text=True, timeout=120)
    print(out.stdout[-3000:])
    assert out.returncode == 0 and "runMoeBlock" in out.stdout and "ALL PASSED" in out.stdout, out.stdout + out.stderr


@pytest.mark.gpu
def test_gpu_gemma4_block_from_gguf_apex(ctx, tmp_path):
    # the whole Gemma4 MoE block from a file: Q8_0 router, Q3_K gate/up and
    # IQ4_NL down experts, every norm vector and the output scale read back
    import pyoracle as orc
    from llmtoy_amd import lib as ltlib
    w = synth.moe_weights(47, 2816, 16, 704, router_type=ggml.Q8_0, gate_up_type=ggml.Q3_K,
                          down_type=ggml.IQ4_NL)
    nm = synth.gemma4_norms(47, 2816, 16)
    r = gguf.GgufReader(write_gemma4_layer(str(tmp_path / "g4.gguf"), w, nm, 0.75))
    L = gguf.load_moe_layer(r, 0)
    norms, los = gguf.load_gemma4_norms(r, 0)
    x, dense = synth.normal(synth.stream(47, 1), (2816,)), synth.normal(synth.stream(47, 2), (2816,))
    tens = lt.upload_moe(ctx, L)
    ids = np.zeros(8, np.uint32)
    got = ltlib.gemma4_moe_block(ctx, x.copy(), dense, *tens, 8, L.d_expert, norms, los, 1e-6, precise=True,
                                 out_ids=ids)
    for t in tens:
        t.free()
    ref, rids, _ = orc.gemma4_moe_block(w, x, dense, 8, nm, 0.75, 1e-6)
    assert ids.tolist() == rids.tolist()
    assert float(np.linalg.norm(got - ref) / np.linalg.norm(ref)) < 1e-3
