"""Deterministic random-init qwen3 GGUF files (ctypes over libmalkin_synth.so, built from synth/synth_gguf.c).

The reference ships no models; its Model reads general.architecture, the qwen3.* keys and the tensors listed in
model.cpp:78-135. The presets below are the BASELINE.json configurations' architectures.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmalkin_synth.so")

F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 1, 8, 12, 13, 14, 30
MIX_UNIFORM, MIX_Q4_K_M = 0, 1


class _Config(ctypes.Structure):
    _fields_ = [
        ("n_layer", ctypes.c_int), ("n_embd", ctypes.c_int), ("n_ff", ctypes.c_int), ("n_head", ctypes.c_int),
        ("n_head_kv", ctypes.c_int), ("head_dim", ctypes.c_int), ("n_vocab", ctypes.c_int),
        ("n_ctx_train", ctypes.c_int), ("rope_base", ctypes.c_float), ("rms_eps", ctypes.c_float),
        ("tied", ctypes.c_int), ("type", ctypes.c_int), ("mix", ctypes.c_int), ("std", ctypes.c_float),
        ("seed", ctypes.c_uint64), ("name", ctypes.c_char * 32), ("eos_id", ctypes.c_int),
    ]


# Qwen3 architectures of the BASELINE.json configurations (E, H, KV, D, F, layers, vocab).
PRESETS = {
    "qwen3-0.6b": dict(n_layer=28, n_embd=1024, n_ff=3072, n_head=16, n_head_kv=8, head_dim=128, n_vocab=151936,
                       tied=True),
    "qwen3-4b": dict(n_layer=36, n_embd=2560, n_ff=9728, n_head=32, n_head_kv=8, head_dim=128, n_vocab=151936,
                     tied=True),
    "qwen3-8b": dict(n_layer=36, n_embd=4096, n_ff=12288, n_head=32, n_head_kv=8, head_dim=128, n_vocab=151936,
                     tied=False),
    "qwen3-14b": dict(n_layer=40, n_embd=5120, n_ff=17408, n_head=40, n_head_kv=8, head_dim=128, n_vocab=151936,
                      tied=False),
    # Small shapes for parity tests (same head layout rules: head_dim 128, GQA).
    "tiny": dict(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=128, n_vocab=1024, tied=False),
    "tiny-tied": dict(n_layer=2, n_embd=512, n_ff=768, n_head=8, n_head_kv=2, head_dim=64, n_vocab=2048, tied=True),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        _lib = ctypes.CDLL(LIB_PATH)
        _lib.mks_write_gguf.argtypes = [ctypes.c_char_p, ctypes.POINTER(_Config), ctypes.c_int]
        _lib.mks_write_gguf.restype = ctypes.c_int
        _lib.mks_file_bytes.argtypes = [ctypes.POINTER(_Config)]
        _lib.mks_file_bytes.restype = ctypes.c_int64
        _lib.mks_quantize_rows.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                           ctypes.c_void_p]
        _lib.mks_quantize_rows.restype = ctypes.c_int
    return _lib


def make_config(preset="tiny", wtype=Q8_0, mix=MIX_UNIFORM, seed=1, std=0.02, rope_base=1e6, rms_eps=1e-6,
                n_ctx_train=40960, eos_id=-1, **over):
    """eos_id >= 0: the file carries tokenizer.ggml.eos_token_id = eos_id (no token list: the synthetic models have
    no tokenizer)."""
    p = dict(PRESETS[preset])
    p.update(over)
    c = _Config()
    for k in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab"):
        setattr(c, k, int(p[k]))
    c.n_ctx_train = n_ctx_train
    c.rope_base = rope_base
    c.rms_eps = rms_eps
    c.tied = 1 if p.get("tied") else 0
    c.type = wtype
    c.mix = mix
    c.std = std
    c.seed = seed
    c.name = preset.encode()[:31]
    c.eos_id = eos_id
    return c


def file_bytes(cfg):
    return int(lib().mks_file_bytes(ctypes.byref(cfg)))


_BLOCK = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def quantize_rows(wtype, x):
    """The writer's quantizer on x [rows][k] float32: GGUF rows of type wtype as uint8 [rows][row bytes]."""
    import numpy as np
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.shape
    qk, bs = _BLOCK[wtype]
    out = np.empty((rows, k // qk * bs), dtype=np.uint8)
    rc = lib().mks_quantize_rows(wtype, x.ctypes.data, rows, k, out.ctypes.data)
    if rc != 0:
        raise ValueError(f"mks_quantize_rows: type {wtype} with {k} columns unsupported")
    return out


def write_gguf(path, cfg, threads=None):
    if threads is None:
        threads = min(16, os.cpu_count() or 1)
    rc = lib().mks_write_gguf(path.encode(), ctypes.byref(cfg), int(threads))
    if rc != 0:
        raise RuntimeError(f"mks_write_gguf({path}) failed: {rc}")
    return path
