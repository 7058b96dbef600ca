"""The C-ABI library loads and exports every symbol include/*.h declares (no compute calls: no GPU needed)."""
import ctypes
import glob
import os
import re

import pytest

import malkin_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    names = set()
    for h in sorted(glob.glob(os.path.join(ROOT, "include", "*.h"))):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(mk_\w+)\s*\(", text))
    return names


def test_library_exports_every_declared_symbol():
    lib = malkin_amd.load()
    names = declared()
    assert len(names) >= 40
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding covers the same surface
    assert names == set(malkin_amd.SIGNATURES)


def test_init_without_device_reports_status():
    lib = malkin_amd.load()
    p = ctypes.c_void_p()
    rc = lib.mk_init(0, ctypes.byref(p))
    if rc == malkin_amd.MK_OK:
        lib.mk_destroy(p)
        pytest.skip("a device is present")
    assert rc == malkin_amd.MK_ERR_NO_DEVICE
    assert b"no HIP device" in lib.mk_last_error()


def test_packed_bytes_keeps_gguf_size():
    lib = malkin_amd.load()
    assert lib.mk_packed_bytes(malkin_amd.Q8_0, 4096, 4096) == 4096 * 4096 // 32 * 34
    assert lib.mk_packed_bytes(malkin_amd.Q4_K, 17408, 5120) == 17408 * 5120 // 256 * 144
    assert lib.mk_packed_bytes(malkin_amd.Q6_K, 5120, 17408) == 5120 * 17408 // 256 * 210
    assert lib.mk_packed_bytes(malkin_amd.Q8_0, 7, 64) == 0  # rows % 8: no layout
    assert lib.mk_packed_bytes(1, 8, 64) == 0  # F16: no device kernel


def test_synthetic_gguf_is_deterministic(synth_lib, tmp_path):
    cfg = synth_lib.make_config("tiny", synth_lib.Q4_K, seed=5)
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    synth_lib.write_gguf(a, cfg, threads=1)
    synth_lib.write_gguf(b, cfg, threads=7)
    assert open(a, "rb").read() == open(b, "rb").read()
    assert os.path.getsize(a) == synth_lib.file_bytes(cfg)
