"""The GGUF reader (mrml_gguf_*, C ABI) and writer, on the CPU.

The reader follows GgufFile::open / read_tensor_bytes
(crates/mrml-tensor/src/gguf.rs:78-184).  The reference ships no GGUF file
and its loader tests fetch one over the network, so the fixtures here are
assembled byte by byte in the tests from the format gguf.rs reads (the
struct packing below is written independently of the package's writer), and
every expectation is a property of that format:
  * header fields, metadata keys in key-byte order (the reference's
    OrderedMap), a repeated key or tensor name keeping its last value;
  * data offset = end of the directory rounded up to general.alignment
    (default 32; gguf.rs:153-163), tensor bytes at data_offset + offset;
  * byte size = numel / block size * block bytes over the first four dims,
    extra dims dropped (gguf.rs:106-147, types.rs:32-70, 179-181);
  * GgufValue::as_u32 / as_f32 conversions (gguf.rs:25-46);
  * the reference's error cases: bad magic, versions outside 2..3, dtype ids
    outside gguf.rs:121-133, unknown value types, non-UTF-8 strings, and
    truncation anywhere in the header.
The writer is then checked by reading back what it wrote, and a random-init
Gemma-2 weight set round-trips bit for bit.
"""

from __future__ import annotations

import struct
from pathlib import Path

import numpy as np
import pytest

MAGIC = 0x46554747


def s(text) -> bytes:
    b = text.encode() if isinstance(text, str) else text
    return struct.pack("<Q", len(b)) + b


def kv(key, vtype, payload: bytes) -> bytes:
    return s(key) + struct.pack("<I", vtype) + payload


def tensor_entry(name, dims, ttype, offset) -> bytes:
    return s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ttype, offset)


def gguf_bytes(kvs: list[bytes], tensors: list[bytes], version=3) -> bytes:
    return struct.pack("<IIQQ", MAGIC, version, len(tensors), len(kvs)) + b"".join(kvs) + b"".join(tensors)


def write(tmp_path, data: bytes, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


def test_header_metadata_and_tensor_known_answer(gguf, tmp_path):
    kvs = [kv("b.key", 8, s("hi")), kv("a.count", 5, struct.pack("<i", 7)),
           kv("general.alignment", 4, struct.pack("<I", 64))]
    head = gguf_bytes(kvs, [tensor_entry("t0", [64, 3], 8, 0), tensor_entry("n", [5], 0, 256)])
    data_off = (len(head) + 63) // 64 * 64
    payload = np.arange(204, dtype=np.uint8)
    norm = np.linspace(-1, 1, 5, dtype=np.float32)
    blob = bytearray(head + b"\0" * (data_off - len(head)) + payload.tobytes())
    blob += b"\0" * (data_off + 256 - len(blob)) + norm.tobytes()
    with gguf.GgufFile(write(tmp_path, bytes(blob))) as g:
        assert g.version == 3 and g.data_offset == data_off
        assert [k for k, _ in g.meta_keys] == ["a.count", "b.key", "general.alignment"]
        assert dict(g.meta_keys) == {"a.count": 5, "b.key": 8, "general.alignment": 4}
        assert g.meta_str("b.key") == "hi" and g.meta_u32("a.count") == 7 and g.meta_u32("b.key") is None
        assert list(g.tensors) == ["n", "t0"]
        t0 = g.tensors["t0"]
        assert (t0["type"], t0["n_dims"], t0["dims"], t0["offset"], t0["size_bytes"]) == (8, 2, [64, 3, 1, 1], 0, 204)
        assert np.array_equal(g.read_tensor_bytes("t0"), payload)
        assert np.array_equal(g.read_tensor_bytes("n").view(np.float32), norm)


def test_default_alignment_and_alignment_value_types(gguf, tmp_path):
    for align_kv, want in ((None, 32), (kv("general.alignment", 10, struct.pack("<Q", 16)), 16),
                           (kv("general.alignment", 1, struct.pack("<b", 64)), 32),  # i8: no as_u32
                           (kv("general.alignment", 5, struct.pack("<i", -64)), 32)):  # negative i32: none
        head = gguf_bytes([align_kv] if align_kv else [], [tensor_entry("x", [8], 0, 0)], version=2)
        off = (len(head) + want - 1) // want * want
        p = write(tmp_path, head + b"\0" * (off - len(head)) + bytes(32))
        with gguf.GgufFile(p) as g:
            assert g.version == 2 and g.data_offset == off, (align_kv, want)


def test_dims_beyond_four_and_zero_dims(gguf, tmp_path):
    head = gguf_bytes([], [tensor_entry("five", [32, 2, 1, 1, 7], 2, 0), tensor_entry("scalar", [], 0, 64)])
    off = (len(head) + 31) // 32 * 32
    p = write(tmp_path, head + b"\0" * (off - len(head) + 128))
    with gguf.GgufFile(p) as g:
        f, sc = g.tensors["five"], g.tensors["scalar"]
        assert f["n_dims"] == 4 and f["dims"] == [32, 2, 1, 1] and f["size_bytes"] == 2 * 18
        assert sc["n_dims"] == 0 and sc["dims"] == [1, 1, 1, 1] and sc["size_bytes"] == 4


@pytest.mark.parametrize("ttype,block,nbytes", [(0, 1, 4), (1, 1, 2), (2, 32, 18), (3, 32, 20), (8, 32, 34),
                                                (12, 256, 144), (13, 256, 176), (14, 256, 210), (16, 256, 136),
                                                (30, 1, 2)])
def test_type_sizes(gguf, tmp_path, ttype, block, nbytes):
    head = gguf_bytes([], [tensor_entry("w", [512, 3], ttype, 0)])
    p = write(tmp_path, head + bytes(4096))
    with gguf.GgufFile(p) as g:
        assert g.tensors["w"]["size_bytes"] == 512 * 3 // block * nbytes


def test_repeated_names_keep_the_last_value(gguf, tmp_path):
    kvs = [kv("k", 4, struct.pack("<I", 1)), kv("k", 4, struct.pack("<I", 2))]
    head = gguf_bytes(kvs, [tensor_entry("t", [32], 0, 0), tensor_entry("t", [64], 0, 128)])
    p = write(tmp_path, head + bytes(512))
    with gguf.GgufFile(p) as g:
        assert g.meta_keys == [("k", 4)] and g.meta_u32("k") == 2
        assert list(g.tensors) == ["t"] and g.tensors["t"]["offset"] == 128 and g.tensors["t"]["size_bytes"] == 256


def test_value_conversions(gguf, tmp_path):
    kvs = [kv("u64", 10, struct.pack("<Q", (1 << 32) + 5)), kv("i64", 11, struct.pack("<q", 9)),
           kv("i64neg", 11, struct.pack("<q", -1)), kv("u16", 2, struct.pack("<H", 300)),
           kv("u8", 0, struct.pack("<B", 200)), kv("i16", 3, struct.pack("<h", 5)),
           kv("f64", 12, struct.pack("<d", 0.1)), kv("u32", 4, struct.pack("<I", 16777217)),
           kv("f32", 6, struct.pack("<f", 1.5)), kv("i32", 5, struct.pack("<i", 3)),
           kv("bool", 7, struct.pack("<B", 2)),
           kv("arr", 9, struct.pack("<IQ", 8, 2) + s("x") + s("yz")),
           kv("nested", 9, struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 4, 3) + struct.pack("<III", 1, 2, 3)),
           kv("empty_unknown", 9, struct.pack("<IQ", 99, 0))]
    p = write(tmp_path, gguf_bytes(kvs, []))
    with gguf.GgufFile(p) as g:
        assert g.meta_u32("u64") == 5 and g.meta_u32("i64") == 9 and g.meta_u32("i64neg") is None
        assert g.meta_u32("u16") == 300 and g.meta_u32("u8") == 200 and g.meta_u32("i16") is None
        assert g.meta_u32("i32") == 3 and g.meta_u32("f32") is None and g.meta_u32("bool") is None
        assert g.meta_f32("f64") == float(np.float32(0.1)) and g.meta_f32("f32") == 1.5
        assert g.meta_f32("u32") == float(np.float32(16777217)) and g.meta_f32("i32") is None
        assert g.meta_array("arr") == (8, 2) and g.meta_array("nested") == (9, 1)
        assert g.meta_array("empty_unknown") == (99, 0) and g.meta_array("u8") is None
        assert g.meta_u32("missing") is None and dict(g.meta_keys)["bool"] == 7


@pytest.mark.parametrize("case,needle", [
    ("magic", "Invalid GGUF magic number: 0x46554746"),
    ("version1", "Unsupported GGUF version: 1"),
    ("version4", "Unsupported GGUF version: 4"),
    ("dtype", "Unsupported GGUF dtype ID: 6"),
    ("vtype", "Unknown GGUF value type ID: 13"),
    ("item", "Unknown GGUF value type ID: 77"),
    ("utf8", "not valid UTF-8"),
    ("bigstr", "runs past the end"),
    # item counts the remaining bytes cannot hold at the items' smallest
    # encoding fail before any item is allocated
    ("bigarr", "array of 150 items"),
    ("bignested", "array of 20 items"),
])
def test_malformed_files_fail_cleanly(gguf, tmp_path, case, needle):
    good_t = [tensor_entry("t", [32], 0, 0)]
    data = {
        "magic": struct.pack("<IIQQ", MAGIC - 1, 3, 0, 0),
        "version1": gguf_bytes([], [], version=1),
        "version4": gguf_bytes([], [], version=4),
        "dtype": gguf_bytes([], [tensor_entry("t", [32], 6, 0)]),  # Q5_0 is not in gguf.rs's table
        "vtype": gguf_bytes([kv("k", 13, b"")], good_t),
        "item": gguf_bytes([kv("k", 9, struct.pack("<IQ", 77, 1) + b"\0")], good_t),
        "utf8": gguf_bytes([kv(b"\xff\xfe", 4, struct.pack("<I", 1))], good_t),
        "bigstr": gguf_bytes([struct.pack("<Q", 1 << 60) + b"k"], good_t),
        "bigarr": gguf_bytes([kv("k", 9, struct.pack("<IQ", 10, 150))], good_t),
        "bignested": gguf_bytes([kv("k", 9, struct.pack("<IQ", 9, 20))], good_t),
    }[case]
    with pytest.raises(gguf.GgufError) as e:
        gguf.GgufFile(write(tmp_path, data + bytes(128)))
    assert e.value.status == -6 and needle in str(e.value)


def test_every_truncation_fails_cleanly(gguf, tmp_path):
    kvs = [kv("general.name", 8, s("tiny")), kv("a", 9, struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2))]
    full = gguf_bytes(kvs, [tensor_entry("t", [32, 2], 2, 0)])
    for n in range(len(full)):
        with pytest.raises(gguf.GgufError) as e:
            gguf.GgufFile(write(tmp_path, full[:n]))
        assert e.value.status == -6, n
    # the whole directory parses; the tensor's bytes are missing
    with gguf.GgufFile(write(tmp_path, full)) as g:
        with pytest.raises(gguf.GgufError) as e:
            g.read_tensor_bytes("t")
        assert e.value.status == -6 and "past the end" in str(e.value)


def test_missing_file_and_names(gguf, tmp_path):
    with pytest.raises(gguf.GgufError) as e:
        gguf.GgufFile(tmp_path / "absent.gguf")
    assert e.value.status == -7
    with gguf.GgufFile(write(tmp_path, gguf_bytes([], []))) as g:
        with pytest.raises(gguf.GgufError):
            g.read_tensor_bytes("nope")
    lib = gguf._lib()
    idx = gguf.ctypes.c_int64()
    assert lib.mrml_gguf_find_tensor(None, b"x", gguf.ctypes.byref(idx)) == -1


def test_writer_layout(gguf, tmp_path):
    rng = np.random.default_rng(3)
    a = rng.integers(0, 256, 3 * 18, dtype=np.uint8)
    b = rng.standard_normal(7).astype(np.float32)
    c = rng.integers(0, 256, 34 * 2, dtype=np.uint8)
    p = tmp_path / "w.gguf"
    gguf.write_gguf(p, [("general.name", gguf.STRING, "w"), ("x.list", gguf.ARRAY, (gguf.INT32, [1, -2, 3]))],
                    [("a", [96], gguf.Q4_0, a), ("b", [7], gguf.F32, b), ("c", [32, 2], gguf.Q8_0, c)],
                    alignment=64)
    raw = p.read_bytes()
    with gguf.GgufFile(p) as g:
        assert g.data_offset % 64 == 0 and g.meta_u32("general.alignment") == 64
        assert g.meta_str("general.name") == "w" and g.meta_array("x.list") == (gguf.INT32, 3)
        for name, want in (("a", a), ("b", b), ("c", c)):
            t = g.tensors[name]
            assert t["offset"] % 64 == 0
            got = g.read_tensor_bytes(name)
            assert np.array_equal(got, want.view(np.uint8))
            start = g.data_offset + t["offset"]
            assert raw[start:start + got.nbytes] == want.tobytes()
    with pytest.raises(ValueError):
        gguf.write_gguf(tmp_path / "bad.gguf", [], [("a", [96], gguf.Q4_0, a[:-1])])


def test_gemma2_round_trip(gguf, synth, tmp_path):
    cfg = dict(n_layers=2, dim=256, n_heads=2, n_kv_heads=1, head_dim=256, ffn_dim=512, vocab=1000, ctx_len=64,
               rope_base=10000.0, eps=1e-6, attn_scale=1.0 / 16.0)
    for tie_q8 in (False, True):
        model = synth.gemma2_model(cfg, seed=11, tie_q8=tie_q8)
        p = tmp_path / f"g{int(tie_q8)}.gguf"
        gguf.write_gemma2(p, model)
        back = gguf.read_gemma2(p)
        for k, v in cfg.items():
            assert np.float32(back["cfg"][k]) == np.float32(v), k
        assert back["tie_q8"] == tie_q8
        assert np.array_equal(back["tok_embd"], model["tok_embd"])
        assert np.array_equal(back["output_norm"], model["output_norm"])
        for L0, L1 in zip(model["layers"], back["layers"]):
            assert L0.keys() == L1.keys()
            for k in L0:
                assert L1[k].dtype == L0[k].dtype and np.array_equal(L1[k], L0[k]), k
        with gguf.GgufFile(p) as g:
            names = set(g.tensors)
            assert {"token_embd.weight", "output_norm.weight", "blk.1.attn_q.weight", "blk.0.ffn_down.weight",
                    "blk.1.post_attention_norm.weight", "blk.0.post_ffw_norm.weight"} <= names
            assert g.tensors["blk.0.ffn_down.weight"]["dims"][:2] == [512, 256]
            assert g.meta_str("general.architecture") == "gemma2" and g.meta_u32("gemma2.block_count") == 2


def _fuzz_seed() -> bytes:
    """A small file with every value type, a nested array and three tensors."""
    kvs = [kv("a.u8", 0, struct.pack("<B", 7)), kv("b.i8", 1, struct.pack("<b", -3)),
           kv("c.u16", 2, struct.pack("<H", 500)), kv("d.i16", 3, struct.pack("<h", -500)),
           kv("e.u32", 4, struct.pack("<I", 70000)), kv("f.i32", 5, struct.pack("<i", -70000)),
           kv("g.f32", 6, struct.pack("<f", 1.5)), kv("h.bool", 7, struct.pack("<B", 1)),
           kv("i.str", 8, s("hello gguf")), kv("j.u64", 10, struct.pack("<Q", 1 << 40)),
           kv("k.i64", 11, struct.pack("<q", -(1 << 40))), kv("l.f64", 12, struct.pack("<d", 2.25)),
           kv("m.arr", 9, struct.pack("<IQ", 8, 3) + s("x") + s("yy") + s("zzz")),
           kv("n.nested", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 4, 2) + struct.pack("<II", 1, 2) +
              struct.pack("<IQ", 6, 1) + struct.pack("<f", 0.5)),
           kv("general.alignment", 4, struct.pack("<I", 32))]
    tensors = [tensor_entry("t.f32", [8, 2], 0, 0), tensor_entry("t.q8", [32, 2], 8, 64),
               tensor_entry("t.q4", [64], 2, 160)]
    head = gguf_bytes(kvs, tensors)
    pad = (-len(head)) % 32
    return head + b"\0" * pad + bytes(range(256)) * 1


def test_reader_mutation_fuzz_under_sanitizers(tmp_path):
    """The reader under AddressSanitizer and UBSan (host code only): 20000
    mutants of a file with every value type, nested arrays and three tensors
    (random byte overwrites, extreme 64-bit lengths, small type ids and
    counts, cuts) are opened and walked completely -- every key's readings,
    every tensor's info, name lookup and bytes.  A memory error, leak or
    undefined behaviour aborts the program, so a clean exit is the check."""
    import shutil
    import subprocess
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    root = Path(__file__).resolve().parents[1]
    exe = tmp_path / "gguf_fuzz"
    r = subprocess.run(["g++", "-O1", "-g", "-std=c++17", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                        str(root / "tests/native/gguf_fuzz.cpp"), str(root / "qt_llama.cpp_amd/csrc/gguf.cpp"),
                        "-I", str(root / "include"), "-o", str(exe)], capture_output=True, text=True)
    if r.returncode != 0 and "asan" in (r.stderr or "").lower():
        pytest.skip("AddressSanitizer runtime not available")
    assert r.returncode == 0, r.stderr[-2000:]
    seed = tmp_path / "seed.gguf"
    seed.write_bytes(_fuzz_seed())
    out = subprocess.run([str(exe), str(seed), str(tmp_path / "mutant.gguf"), "20000", "7"], capture_output=True,
                         text=True, timeout=600, env={"ASAN_OPTIONS": "detect_leaks=1"})
    assert out.returncode == 0, (out.stdout[-500:], out.stderr[-3000:])
    fields = out.stdout.split()
    assert fields[0] == "ok" and int(fields[1]) == 20000 and int(fields[2]) > 1000, out.stdout
