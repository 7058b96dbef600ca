"""The synthetic model writer (malkin_amd/synth): every quantized weight dequantizes (by the CPU oracle's
dequantize_row, the reference's block formats) to the N(0, 0.02) it was drawn from, norms to about 1, and files are
byte-identical across writes and thread counts. A quantizer that writes zero scales (as a subnormal half scale read
back as zero once did for Q6_K) fails here."""
import hashlib
import os

import numpy as np
import pytest

from gguf_read import Gguf


def digest(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


@pytest.mark.parametrize("wtype,mix", [(8, 0), (12, 0), (13, 0), (14, 0), (12, 1), (1, 0), (30, 0)])
def test_weights_have_the_drawn_spread(tmp_path, synth_lib, oracle, wtype, mix):
    synth = synth_lib
    path = str(tmp_path / "m.gguf")
    synth.write_gguf(path, synth.make_config("tiny", wtype, mix=mix, seed=3), threads=2)
    g = Gguf(path)
    assert g.kv["general.architecture"] == "qwen3"
    types = set()
    for name in g.tensors:
        ty, cols, rows = g.rows(name)
        vals = np.concatenate([oracle.dequantize_row(ty, rows[r], cols) for r in range(min(8, len(rows)))])
        if name.endswith("norm.weight"):
            assert ty == 0 and abs(vals.mean() - 1.0) < 0.05, name
            continue
        types.add(ty)
        sd = float(vals.std())
        assert 0.018 < sd < 0.022, (name, ty, sd)
        assert abs(float(vals.mean())) < 0.004, (name, ty)
    if mix == 1:
        assert types == {12, 14}  # Q4_K_M: Q4_K with Q6_K output / attn_v / ffn_down
    else:
        assert types == {wtype}


def test_files_are_deterministic(tmp_path, synth_lib):
    synth = synth_lib
    a, b = str(tmp_path / "a.gguf"), str(tmp_path / "b.gguf")
    cfg = synth.make_config("tiny", 14, seed=9)
    synth.write_gguf(a, cfg, threads=1)
    synth.write_gguf(b, cfg, threads=4)
    assert os.path.getsize(a) == synth.file_bytes(cfg)
    assert digest(a) == digest(b)
