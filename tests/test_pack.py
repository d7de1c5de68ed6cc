"""The pack reader (src/pack.rs): a written pack reads back entry by entry, and damaged or
inconsistent packs are refused with the reference's messages. Host code only, no GPU."""
import json
import os
import struct

import numpy as np
import pytest

from packs import PackWriter, sample_pack, sample_weights


@pytest.fixture(scope="module")
def tm():
    import telmo_amd

    return telmo_amd


@pytest.fixture(scope="module")
def sample(tm):
    return sample_pack(lambda w, n, k, p: tm.encode(w, n, k, tm.Precision(p)))


def refused(tm, data, message):
    with pytest.raises(tm.TelmoError) as e:
        tm.Pack.from_bytes(data)
    assert message in str(e.value), str(e.value)


def test_a_file_pack_reads_back(tm, sample, tmp_path):
    path = tmp_path / "model.pack"
    path.write_bytes(sample)
    for pack in (tm.Pack.open(str(path)), tm.Pack.from_bytes(sample)):
        assert pack.model() == "test"
        assert pack.meta("source") == "x" and pack.meta("missing") is None
        assert pack.metadata() == [("source", "x")]
        names = [e.name for e in pack.entries()]
        assert names == ["w8", "wq", "wh", "bias", "config.json"]
        w = sample_weights().reshape(40, 64)
        for name, prec in (("w8", 3), ("wq", 4), ("wh", 1)):
            values, scales = pack.matrix_parts(name)
            want_v, want_s = tm.encode(w, 40, 64, tm.Precision(prec))
            assert np.array_equal(values, want_v)
            assert (scales is None and want_s.size == 0) or np.array_equal(scales, want_s)
            rows = tm.decode(values, scales if scales is not None else np.zeros(0, np.float32), 40, 64,
                             tm.Precision(prec))
            assert np.array_equal(rows, tm.decode(want_v, want_s, 40, 64, tm.Precision(prec)))
        assert np.array_equal(pack.vector("bias", [2, 3]), np.arange(1, 7, dtype=np.float32).reshape(2, 3))
        with pytest.raises(tm.TelmoError, match=r"has shape \[2, 3\], and the model needs \[6\]"):
            pack.vector("bias", [6])
        assert pack.bytes("config.json") == b'{"a":1}'
        with pytest.raises(tm.TelmoError, match="Entry missing is missing"):
            pack.bytes("missing")
        with pytest.raises(tm.TelmoError, match="isn't a bytes entry"):
            pack.bytes("w8")
        assert pack.precision() is None  # int8, Q8_0 and f16 mixed
        assert pack.data_bytes() == sum(e.size() for e in pack.entries())
    assert tm.Pack.open(str(path)).is_mapped()
    assert not tm.Pack.from_bytes(sample).is_mapped()


def test_entries_are_64_byte_aligned_views(tm, sample, tmp_path):
    import ctypes

    from telmo_amd import _lib
    from telmo_amd.pack import _Entry

    path = tmp_path / "a.pack"
    path.write_bytes(sample)
    pack = tm.Pack.open(str(path))
    for i in range(len(pack.entries())):
        e = _Entry()
        assert _lib.lib().tg_pack_entry_at(pack._h, i, ctypes.byref(e)) == 0
        assert e.data % 64 == 0
        if e.scales:
            assert e.scales % 64 == 0


def test_damaged_packs_are_refused(tm, sample):
    tm.Pack.from_bytes(sample)
    refused(tm, sample[:-1], "Its index is missing")
    wrong_version = bytearray(sample)
    wrong_version[8] = 2
    refused(tm, bytes(wrong_version), "The pack has format version 2, and this version of the engine reads 1.")
    no_magic = bytearray(sample)
    no_magic[0] = 0
    refused(tm, bytes(no_magic), "It isn't a pack.")
    refused(tm, sample[:30], "It isn't a pack.")
    moved = bytearray(sample)
    at, n = struct.unpack("<QQ", moved[-24:-8])
    moved[-24:-16] = struct.pack("<Q", at + 1)
    refused(tm, bytes(moved), "Its index is out of place.")


def index_of(data):
    at, n = struct.unpack("<QQ", data[-24:-8])
    return data[:at], json.loads(data[at:at + n])


def rewrite(head, root):
    text = json.dumps(root, separators=(",", ":")).encode()
    return bytes(head + text + struct.pack("<QQ", len(head), len(text)) + b"TELMOIDX")


@pytest.mark.parametrize("edit,message", [
    (lambda r: r.pop("model"), "The index names no model."),
    (lambda r: r.pop("entries"), "The index lists no entries."),
    (lambda r: r["metadata"].update(bad=3), "A metadata value isn't a string."),
    (lambda r: r["entries"][0].pop("name"), "An entry has no name."),
    (lambda r: r["entries"][0].update(type="tensor"), "Entry w8 has an unknown type."),
    (lambda r: r["entries"][0].update(precision="int4"), "Entry w8 has an unknown precision."),
    (lambda r: r["entries"][0].update(n=0), "Entry w8 has an impossible shape."),
    (lambda r: r["entries"][1].update(k=48), "Entry wq has an impossible shape."),
    (lambda r: r["entries"][0].update(n=60), "Entry w8 has the wrong size."),
    (lambda r: r["entries"][0].update(n=-1), "Entry w8 has no valid n."),
    (lambda r: r["entries"][0].update(offset=r["entries"][0]["offset"] + 4), "Entry w8 is out of place."),
    (lambda r: r["entries"][0].update(offset=0), "Entry w8 is out of place."),
    (lambda r: r["entries"][0].update(scales_bytes=4), "Entry w8 has the wrong number of scales."),
    (lambda r: r["entries"][2].update(offset=r["entries"][0]["offset"]), "Two entries overlap."),
    (lambda r: r["entries"][3].update(shape=[6, 1, 1, 1, 1, 1, 1, 1, 1]), "Entry bias has no valid shape."),
    (lambda r: r["entries"][3].update(shape=[7]), "Entry bias has the wrong size."),
    (lambda r: r["entries"][4].update(name="w8"), "Two entries are named w8."),
])
def test_inconsistent_indexes_are_refused(tm, sample, edit, message):
    head, root = index_of(sample)
    edit(root)
    refused(tm, rewrite(head, root), message)


@pytest.mark.parametrize("text,message", [
    (b'{"model":"a","model":"b","entries":[]}', "duplicate key"),
    (b'{"model":"\\ud800","entries":[]}', "unpaired surrogate"),
    (b'{"model":"a","entries":[]} x', "text after the value"),
    (b'{"model":"a\x01","entries":[]}', "control character in a string"),
    (b'{"model":"\xff","entries":[]}', "invalid UTF-8 in a string"),
    (b'[' * 200 + b']' * 200, "nested too deeply"),
    (b'{"model":"a","entries":[01]}', "expected , or ]"),
])
def test_bad_json_is_refused(tm, sample, text, message):
    head, _ = index_of(sample)
    data = bytes(head + text + struct.pack("<QQ", len(head), len(text)) + b"TELMOIDX")
    refused(tm, data, message)


def test_an_index_in_other_valid_json_reads(tm, sample):
    head, root = index_of(sample)
    text = json.dumps(root, indent=2, ensure_ascii=True).replace('"test"', '"t\\u00e9st"').encode()
    pack = tm.Pack.from_bytes(bytes(head + text + struct.pack("<QQ", len(head), len(text)) + b"TELMOIDX"))
    assert pack.model() == "tést"


def test_the_committed_sample_pack_is_what_the_writer_makes(tm, sample):
    path = os.path.join(os.path.dirname(__file__), "golden", "sample.pack")
    with open(path, "rb") as f:
        assert f.read() == sample


def test_the_reader_survives_mutated_packs_under_sanitizers(tmp_path):
    """Mutation fuzzing of the host-side pack reader (tests/fuzz_pack.cpp) built with g++'s
    AddressSanitizer and UndefinedBehaviorSanitizer: 20,000 damaged variants of three packs
    (int8, f32 and Q8_0 matrices, f32 tensors, bytes, metadata), each refused or walked entry by
    entry without a memory error."""
    import shutil
    import subprocess

    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    here = os.path.dirname(os.path.abspath(__file__))
    csrc = os.path.join(here, "..", "telmo_amd", "csrc")
    exe = str(tmp_path / "fuzz_pack")
    build = subprocess.run([gxx, "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
                            "-o", exe, os.path.join(here, "fuzz_pack.cpp"), os.path.join(csrc, "pack.cpp"),
                            os.path.join(csrc, "layout.cpp")], capture_output=True, text=True)
    if build.returncode != 0:
        pytest.skip("no sanitizer runtime: " + build.stderr[-300:])
    rng = np.random.default_rng(1)
    seeds = []
    w = PackWriter("parakeet-tdt", [("vocab", "8193"), ("note", "x")])
    w.matrix("layers.0.ff1.up", rng.integers(0, 255, 64 * 32, dtype=np.uint8), rng.random(32).astype(np.float32),
             3, 32, 64)
    w.f32("norm.gamma", (16,), rng.random(16))
    w.bytes_entry("tokenizer", b"abc" * 10)
    seeds.append(w.finish())
    w = PackWriter("granite", [])
    w.matrix("w8", sample_weights().tobytes(), None, 0, 40, 64)
    seeds.append(w.finish())
    w = PackWriter("m", [("a", "b")])
    w.matrix("q", rng.integers(0, 255, 64 * 16, dtype=np.uint8), rng.random(2 * 16).astype(np.float32), 4, 16, 64)
    seeds.append(w.finish())
    paths = []
    for i, data in enumerate(seeds):
        p = tmp_path / f"seed{i}.bin"
        p.write_bytes(data)
        paths.append(str(p))
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1", UBSAN_OPTIONS="halt_on_error=1")
    run = subprocess.run([exe, "20000"] + paths, capture_output=True, text=True, env=env, timeout=300)
    assert run.returncode == 0, run.stdout[-500:] + run.stderr[-2000:]
    assert "iterations 20000" in run.stdout
