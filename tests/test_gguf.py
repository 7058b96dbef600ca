"""The host GGUF reader (malkin_amd/csrc/host/gguf.cpp) through mk_gguf_inspect, on the CPU: a synthetic model reads
back with the same directory as an independent Python reader, and malformed files fail with a reason instead of
reading out of bounds (truncation anywhere, bad magic or version, rank 0 or above 4, zero alignment, offsets that
overflow or leave the file, unknown types, duplicate names)."""
import os
import struct

import numpy as np
import pytest

import malkin_amd
from gguf_read import Gguf


def s(text):
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def gguf_bytes(tensors, meta=(), version=3, magic=0x46554747, align=32, pad_data=True):
    """tensors: (name, dims, type, offset, data bytes). meta: (key, type, packed value)."""
    out = struct.pack("<IIQQ", magic, version, len(tensors), len(meta))
    for key, t, val in meta:
        out += s(key) + struct.pack("<I", t) + val
    for name, dims, ty, off, _ in tensors:
        out += s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", ty, off)
    if pad_data:
        out += b"\0" * ((-len(out)) % align)
        data = bytearray()
        for _, _, _, off, blob in tensors:
            if len(data) < off:
                data += b"\0" * (off - len(data))
            data[off:off + len(blob)] = blob
        out += bytes(data)
    return out


def inspect(tmp_path, blob, name="f.gguf"):
    p = str(tmp_path / name)
    with open(p, "wb") as f:
        f.write(blob)
    return malkin_amd.gguf_inspect(p)


def fails(tmp_path, blob, words):
    with pytest.raises(malkin_amd.MkError) as e:
        inspect(tmp_path, blob)
    msg = str(e.value)
    assert any(w in msg for w in words), msg


F32 = 0
ONE = [("a", [8], F32, 0, b"\1" * 32)]


def test_synthetic_model_directory(tmp_path, synth_lib):
    p = str(tmp_path / "m.gguf")
    synth_lib.write_gguf(p, synth_lib.make_config("tiny", 12, mix=1, seed=2), threads=2)
    info = malkin_amd.gguf_inspect(p)
    g = Gguf(p)
    assert info["arch"] == "qwen3" and info["n_layer"] == 2
    assert info["n_tensors"] == len(g.tensors)
    assert info["tensor_bytes"] == sum(g.rows(n)[2].size for n in g.tensors)


def test_minimal_file_and_metadata_kinds(tmp_path):
    meta = [("general.architecture", 8, s("qwen3")), ("qwen3.block_count", 4, struct.pack("<I", 3)),
            ("x.f", 6, struct.pack("<f", 0.5)), ("x.b", 7, b"\1"), ("x.arr", 9, struct.pack("<IQ", 8, 2) + s("p") + s("q")),
            ("x.nested", 9, struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 4, 2) + b"\0" * 8)]
    info = inspect(tmp_path, gguf_bytes(ONE, meta))
    assert info == {"n_tensors": 1, "tensor_bytes": 32, "n_layer": 3, "arch": "qwen3"}


def test_truncation_anywhere_is_an_error(tmp_path):
    blob = gguf_bytes(ONE, [("general.architecture", 8, s("qwen3"))])
    inspect(tmp_path, blob)
    for cut in list(range(0, 80, 3)) + [len(blob) - 1]:
        fails(tmp_path, blob[:cut], ["too short", "past the end", "outside the file"])


def test_bad_magic_and_version(tmp_path):
    fails(tmp_path, gguf_bytes(ONE, magic=0x46554748), ["bad magic"])
    fails(tmp_path, gguf_bytes(ONE, version=2), ["version 2"])


@pytest.mark.parametrize("dims", [[], [2, 2, 2, 2, 1]])
def test_tensor_rank_outside_1_to_4(tmp_path, dims):
    fails(tmp_path, gguf_bytes([("a", dims, F32, 0, b"")]), ["rank"])


def test_zero_alignment(tmp_path):
    blob = gguf_bytes(ONE, [("general.alignment", 4, struct.pack("<I", 0))])
    fails(tmp_path, blob, ["general.alignment"])


def test_tensor_outside_the_file(tmp_path):
    fails(tmp_path, gguf_bytes([("a", [8], F32, 64, b"")]), ["outside the file"])
    # an offset that would wrap start + offset + bytes around 2^64
    blob = gguf_bytes([("a", [8], F32, 2**64 - 16, b"")], pad_data=False)
    blob += b"\0" * ((-len(blob)) % 32) + b"\0" * 64
    fails(tmp_path, blob, ["outside the file"])
    # an element count whose byte size overflows
    fails(tmp_path, gguf_bytes([("a", [2**62, 8], F32, 0, b"")]), ["too many elements", "too large"])


def test_unknown_type_and_partial_block(tmp_path):
    fails(tmp_path, gguf_bytes([("a", [8], 99, 0, b"")]), ["unknown ggml type"])
    fails(tmp_path, gguf_bytes([("a", [33], 8, 0, b"")]), ["whole number of blocks"])


def test_duplicate_tensor_and_missing_file(tmp_path):
    fails(tmp_path, gguf_bytes([("a", [8], F32, 0, b"\0" * 32), ("a", [8], F32, 32, b"\0" * 32)]), ["twice"])
    with pytest.raises(malkin_amd.MkError) as e:
        malkin_amd.gguf_inspect(str(tmp_path / "absent.gguf"))
    assert "open failed" in str(e.value)


def test_no_descriptor_leak_on_errors(tmp_path):
    blob = gguf_bytes(ONE, version=2)
    before = len(os.listdir("/proc/self/fd"))
    for _ in range(50):
        with pytest.raises(malkin_amd.MkError):
            inspect(tmp_path, blob)
    assert len(os.listdir("/proc/self/fd")) <= before + 1


def str_array(items):
    return struct.pack("<IQ", 8, len(items)) + b"".join(s(t) for t in items)


def i32_array(vals):
    return struct.pack("<IQ", 5, len(vals)) + b"".join(struct.pack("<i", v) for v in vals)


def test_end_of_generation_ids(tmp_path):
    """The end-of-generation set of tokenizer.cpp:93-102: the eos / eot / eom ids, plus the control tokens (type 3)
    among the end-of-turn names. A name that is present but not a control token, and ids of other keys, are not in
    it; repeated ids appear once, ascending."""
    toks = ["a", "<|im_end|>", "b", "<|endoftext|>", "<|eot_id|>", "<end_of_turn>", "c"]
    types = [1, 3, 1, 3, 1, 3, 1]  # <|eot_id|> is a normal token here
    meta = [("general.architecture", 8, s("qwen3")),
            ("tokenizer.ggml.eos_token_id", 4, struct.pack("<I", 6)),
            ("tokenizer.ggml.eot_token_id", 4, struct.pack("<I", 3)),
            ("tokenizer.ggml.bos_token_id", 4, struct.pack("<I", 2)),
            ("tokenizer.ggml.tokens", 9, str_array(toks)),
            ("tokenizer.ggml.token_type", 9, i32_array(types))]
    info = inspect(tmp_path, gguf_bytes(ONE, meta))
    assert info["eog"] == [1, 3, 5, 6]
    # Without token types only the metadata ids count; without any of the keys there is no set.
    info = inspect(tmp_path, gguf_bytes(ONE, meta[:3] + meta[4:5]), name="g.gguf")
    assert info["eog"] == [3, 6]
    assert "eog" not in inspect(tmp_path, gguf_bytes(ONE, meta[:1]), name="h.gguf")
    # eom alone, as a u64.
    info = inspect(tmp_path, gguf_bytes(ONE, [("tokenizer.ggml.eom_token_id", 10, struct.pack("<Q", 9))]), name="i.gguf")
    assert info["eog"] == [9]


def test_synthetic_eos_id(tmp_path, synth_lib):
    p = str(tmp_path / "m.gguf")
    synth_lib.write_gguf(p, synth_lib.make_config("tiny", 8, seed=2, eos_id=77), threads=2)
    assert malkin_amd.gguf_inspect(p)["eog"] == [77]
    synth_lib.write_gguf(p, synth_lib.make_config("tiny", 8, seed=2), threads=2)
    assert "eog" not in malkin_amd.gguf_inspect(p)
