"""GGUF files (CPU only): the library's reader against files written by tests/gguf_writer.py.

Mirrors the reference's loader contract (dynalm/src/loader/gguf/gguf.cpp:248-343,
gguf_model.cpp:291-331): directory and metadata read back exactly; split models open
from their first part; every malformed file (truncations, bad magic / version /
alignment / offsets / dims / types, random byte mutations as the reference's parser
fuzzer makes them, dynalm/tests/test_fuzz_parsers.cpp:82-115) is refused with a status
code and never read past its end. No GPU work: uploads are checked in the GPU suite.
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

import dynalm_amd as dq
from dqtest import gguf_weights
from gguf_writer import (ARR, BOOL, F32, F64, GGML_F32, GGML_Q4_0, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, I8, I32, I64,
                         STR, U8, U16, U32, U64, GgufWriter, split_names)
from oracle import oracle as O


def model(version: int = 3, alignment: int | None = 64) -> tuple[GgufWriter, dict[str, bytes]]:
    w = GgufWriter(version, alignment)
    w.kv("general.architecture", STR, "llama").kv("llama.block_count", U32, 2).kv("small", U8, 7)
    w.kv("mid", U16, 513).kv("big", U64, 1 << 40).kv("signed_ok", I32, 12).kv("neg", I64, -3)
    w.kv("ratio", F32, 0.5).kv("precise", F64, 1e-300).kv("flag", BOOL, 1).kv("tiny", I8, -1)
    w.kv("tokens", ARR, (STR, ["a", "bc", ""])).kv("nested", ARR, (ARR, [(I32, [1, 2]), (U8, [3])]))
    blobs = {
        "blk.0.ffn_gate.weight": (GGML_Q4_K, [96, 512], gguf_weights(O.Q4_K, 96, 512, 1).tobytes()),
        "blk.0.ffn_down.weight": (GGML_Q6_K, [64, 768], gguf_weights(O.Q6_K, 64, 768, 2).tobytes()),
        "blk.0.attn_q.weight": (GGML_Q8_0, [40, 96], gguf_weights(O.Q8_0, 40, 96, 3).tobytes()),
        "blk.0.attn_k.weight": (GGML_Q4_0, [24, 160], gguf_weights(O.Q4_0, 24, 160, 4).tobytes()),
        "blk.0.attn_norm.weight": (GGML_F32, [512], np.linspace(0, 1, 512, dtype=np.float32).tobytes()),
        "blk.0.ffn_up_exps.weight": (GGML_Q4_K, [3, 32, 256], gguf_weights(O.Q4_K, 96, 256, 5).tobytes()),
    }
    for name, (t, shape, data) in blobs.items():
        w.tensor(name, t, shape, data)
    return w, {k: v[2] for k, v in blobs.items()}


def write(tmp_path, name: str, data: bytes) -> str:
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def status(path: str) -> str:
    try:
        dq.GgufFile.open(path).close()
    except dq.DqError as e:
        return e.status
    return "ok"


@pytest.mark.parametrize("version", [2, 3])
@pytest.mark.parametrize("alignment", [None, 64, 4096])
def test_directory_and_metadata(tmp_path, version, alignment):
    w, blobs = model(version, alignment)
    with dq.GgufFile.open(write(tmp_path, "m.gguf", w.to_bytes())) as g:
        info = g.info()
        assert info == {"version": version, "alignment": alignment or 32, "n_tensors": len(blobs), "n_parts": 1}
        for name, gtype, shape, data in w.tensors:
            i = g.find(name)
            t = g.tensor(i)
            assert t.name.decode() == name and t.ggml_type == gtype and t.shape == tuple(shape)
            assert t.nbytes == len(data) and t.offset % (alignment or 32) == 0 and t.part == 0
            assert t.dtype == {GGML_Q4_K: O.Q4_K, GGML_Q6_K: O.Q6_K, GGML_Q8_0: O.Q8_0, GGML_Q4_0: O.Q4_0}.get(gtype, -1)
            assert g.data(name) == data
        assert g.find("nope") == -1
        assert g.get_string("general.architecture") == "llama"
        assert [g.get_uint(k) for k in ("llama.block_count", "small", "mid", "big", "signed_ok")] == [2, 7, 513, 1 << 40, 12]
        for key, want in (("neg", "invalid_argument"), ("ratio", "invalid_argument"), ("missing", "not_found"),
                          ("tiny", "invalid_argument")):
            with pytest.raises(dq.DqError) as e:
                g.get_uint(key)
            assert e.value.status == want, key
        with pytest.raises(dq.DqError) as e:
            g.get_string("small")
        assert e.value.status == "invalid_argument"


def test_split_model(tmp_path):
    w, blobs = model()
    names = split_names("tiny", 3)
    paths = [write(tmp_path, n, b) for n, b in zip(names, w.split(3))]
    with dq.GgufFile.open(paths[0]) as g:
        assert g.info()["n_parts"] == 3 and g.info()["n_tensors"] == len(blobs)
        assert sorted({t.part for t in g.tensors()}) == [0, 1, 2]
        for name, data in blobs.items():
            assert g.data(name) == data
        assert g.get_string("general.architecture") == "llama"
    assert status(paths[1]) == "invalid_argument"          # not the first part
    (tmp_path / names[2]).unlink()
    assert status(paths[0]) == "not_found"                 # a missing part
    renamed = write(tmp_path, "tiny.gguf", (tmp_path / names[0]).read_bytes())
    assert status(renamed) == "invalid_argument"           # first part under another name
    # split.tensors.count that disagrees with the parts
    w2, _ = model()
    names2 = split_names("bad", 2)
    p0 = GgufWriter(3, 64)
    p0.kvs = list(w2.kvs)
    p0.kv("split.no", U16, 0).kv("split.count", U16, 2).kv("split.tensors.count", I32, 99)
    p0.tensors = w2.tensors[:3]
    p1 = GgufWriter(3, 64)
    p1.kv("split.no", U16, 1).kv("split.count", U16, 2).kv("split.tensors.count", I32, 99)
    p1.tensors = w2.tensors[3:]
    write(tmp_path, names2[0], p0.to_bytes())
    write(tmp_path, names2[1], p1.to_bytes())
    assert status(str(tmp_path / names2[0])) == "corrupt"
    # a part that names another position
    p1b = GgufWriter(3, 64)
    p1b.kv("split.no", U16, 0).kv("split.count", U16, 2)
    p1b.tensors = w2.tensors[3:]
    p0.kvs = [kv for kv in p0.kvs if kv[0] != "split.tensors.count"]
    write(tmp_path, names2[0], p0.to_bytes())
    write(tmp_path, names2[1], p1b.to_bytes())
    assert status(str(tmp_path / names2[0])) == "corrupt"


def test_malformed_files(tmp_path):
    w, _ = model()
    good = w.to_bytes()
    cases = {
        "magic": (b"GGUX" + good[4:], "corrupt"),
        "v1": (good[:4] + struct.pack("<I", 1) + good[8:], "unsupported"),
        "v4": (good[:4] + struct.pack("<I", 4) + good[8:], "unsupported"),
        "empty": (b"", "corrupt"),
        "counts": (good[:8] + struct.pack("<QQ", 1 << 40, 3) + good[24:], "corrupt"),
    }
    for name, (data, want) in cases.items():
        assert status(write(tmp_path, name + ".gguf", data)) == want, name
    # directory-level faults
    first = w.tensors[0][0]
    bad = {
        "misaligned": w.to_bytes(offsets={first: 8}),
        "past_end": w.to_bytes(offsets={first: 1 << 30}),
        "zero_dims": w.to_bytes(raw_dims={first: []}),
        "five_dims": w.to_bytes(raw_dims={first: [256, 1, 1, 1, 1]}),
        "ragged_row": w.to_bytes(raw_dims={first: [100, 96]}),
        "overflow": w.to_bytes(raw_dims={first: [256, 1 << 62, 1 << 10]}),
    }
    for name, data in bad.items():
        assert status(write(tmp_path, name + ".gguf", data)) == "corrupt", name
    wt = GgufWriter(3)
    wt.tensor("x", 4, [1, 32], b"\0" * 18)                 # ggml id 4: no such type
    assert status(write(tmp_path, "type4.gguf", wt.to_bytes())) == "unsupported"
    wt = GgufWriter(3)
    wt.tensor("x", 100, [1, 32], b"\0" * 18)
    assert status(write(tmp_path, "type100.gguf", wt.to_bytes())) == "unsupported"
    for key, vt, v in (("general.alignment", U32, 48), ("general.alignment", U32, 0), ("general.alignment", STR, "x"),
                       ("general.alignment", I32, -64)):
        wa = GgufWriter(3)
        wa.kv(key, vt, v)
        assert status(write(tmp_path, "align.gguf", wa.to_bytes())) == "corrupt", (vt, v)
    wd = GgufWriter(3).kv("a", U8, 1).kv("a", U8, 2)
    assert status(write(tmp_path, "dupkey.gguf", wd.to_bytes())) == "corrupt"
    wd = GgufWriter(3).tensor("t", GGML_F32, [4], b"\0" * 16).tensor("t", GGML_F32, [4], b"\0" * 16)
    assert status(write(tmp_path, "duptensor.gguf", wd.to_bytes())) == "corrupt"
    wb = GgufWriter(3).kv("b", BOOL, 2)
    assert status(write(tmp_path, "bool.gguf", wb.to_bytes())) == "corrupt"
    wn = GgufWriter(3).kv("deep", ARR, (ARR, [(ARR, [(U8, [1])])]))
    assert status(write(tmp_path, "deep.gguf", wn.to_bytes())) == "corrupt"
    raw = GgufWriter(3).kv("v", U8, 1).to_bytes()             # value type 13: no such type
    k = raw.index(b"v") + 1
    assert status(write(tmp_path, "vtype.gguf", raw[:k] + struct.pack("<I", 13) + raw[k + 4:])) == "corrupt"


def test_every_truncation_is_refused(tmp_path):
    """Each prefix of a valid file is refused (the directory's lengths are checked against the mapping)."""
    w = GgufWriter(3, 32)
    w.kv("general.architecture", STR, "llama").kv("tokens", ARR, (STR, ["ab", "c"]))
    w.tensor("w", GGML_Q8_0, [2, 32], gguf_weights(O.Q8_0, 2, 32, 9).tobytes())
    full = w.to_bytes()
    path = str(tmp_path / "t.gguf")
    for n in range(len(full)):
        with open(path, "wb") as f:
            f.write(full[:n])
        assert status(path) in ("corrupt",), n
    with open(path, "wb") as f:
        f.write(full)
    assert status(path) == "ok"


def test_random_mutations_never_crash(tmp_path):
    """Seeded byte mutations of a valid file: every open returns a status (ok or an error code);
    files that still open keep their tensors inside the file."""
    w, _ = model(alignment=32)
    base = bytearray(w.to_bytes())
    rng = np.random.default_rng(2024)
    path = str(tmp_path / "fuzz.gguf")
    seen = set()
    for _ in range(1500):
        b = bytearray(base)
        for _ in range(int(rng.integers(1, 8))):
            pos = int(rng.integers(0, min(len(b), 1200)))
            b[pos] = int(rng.integers(0, 256))
        if rng.random() < 0.2:
            b = b[:int(rng.integers(0, len(b)))]
        with open(path, "wb") as f:
            f.write(bytes(b))
        st = status(path)
        seen.add(st)
        if st == "ok":
            with dq.GgufFile.open(path) as g:
                for t in g.tensors():
                    assert t.offset + t.nbytes <= len(b)
    assert "ok" in seen and "corrupt" in seen


def test_upload_refusals_without_gpu(tmp_path):
    """Tensors that are not weights of the four types are refused before any device work."""
    w, _ = model()
    w.tensor("vec", GGML_Q8_0, [64], gguf_weights(O.Q8_0, 2, 32, 1).tobytes())
    with dq.GgufFile.open(write(tmp_path, "m.gguf", w.to_bytes())) as g:
        with pytest.raises(dq.DqError) as e:
            g.upload("blk.0.attn_norm.weight")
        assert e.value.status == "unsupported"
        with pytest.raises(dq.DqError) as e:
            g.upload("vec")
        assert e.value.status == "invalid_argument"
        with pytest.raises(dq.DqError) as e:
            g.upload("missing")
        assert e.value.status == "not_found"
