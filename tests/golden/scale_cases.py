"""The BASELINE.json model-level configurations (3, 4, 5) as parity cases at full size.

Shared by tests/golden/make_golden_scale.py (which runs the reference's own hot path, oracle/_ref, on them and writes
scale.npz) and by tests/test_gpu_scale.py (which runs the device library on the same inputs and compares). Each model
is a synthetic GGUF regenerated bit-identically by malkin_amd/synth from the config below; its digest is recorded.

Logit rows are compared through a SHA-256 of their float32 bytes (bit-exact check), with the top entries and a strided
sample kept for diagnosis when a digest differs.
"""
import concurrent.futures as cf
import hashlib
import mmap
import os

import numpy as np

VOCAB = 151936
N_CTX = 4096

MODELS = {
    # config 3: random-init Qwen3-4B, all matmuls Q8_0, tied embeddings
    "c3": dict(preset="qwen3-4b", wtype=8, mix=0, seed=31),
    # config 4: random-init Qwen3-8B, Q8_0, untied LM head (the model bench.py measures)
    "c4": dict(preset="qwen3-8b", wtype=8, mix=0, seed=1),
    # config 5: target Qwen3-14B Q6_K, draft Qwen3-0.6B Q4_K_M (Q4_K with Q6_K attn_v / ffn_down / LM head)
    "c5t": dict(preset="qwen3-14b", wtype=14, mix=0, seed=5),
    "c5d": dict(preset="qwen3-0.6b", wtype=12, mix=1, seed=6),
}

C3_PROMPT, C3_GEN = 512, 128
C4_SEQS, C4_GEN, C4_MIN, C4_MAX = 8, 128, 256, 1024
C5_PREFIX, C5_DRAFT, C5_GEN = 2048, 8, 64
CHUNK = 256  # prompt tokens per forward (the reference engine's kMaxBatch)
SAMPLE_STRIDE = 64


def c3_prompt():
    return np.random.default_rng(303).integers(0, VOCAB, size=C3_PROMPT).astype(np.int32)


def c4_prompts():
    rng = np.random.default_rng(404)
    lens = rng.integers(C4_MIN, C4_MAX + 1, size=C4_SEQS)
    return [rng.integers(0, VOCAB, size=int(n)).astype(np.int32) for n in lens]


def c5_prompt():
    return np.random.default_rng(505).integers(0, VOCAB, size=C5_PREFIX).astype(np.int32)


def tree_batch(root, chain, alt, P, seq=0):
    """The engine's greedy verification layout (engine.cpp:359-381): [next, chain0, alt0, chain1, alt1, ...] at KV
    rows P, P + 1, ...; chain i and alt i sit at RoPE position P + 1 + i under chain i - 1 (the root for i = 0).
    Rows: (id, seq, pos, logits, kv, parent)."""
    rows = [(int(root), seq, P, 1, -1, -1)]
    for i, (c, a) in enumerate(zip(chain, alt)):
        par = 0 if i == 0 else 2 * i - 1
        rows.append((int(c), seq, P + 1 + i, 1, P + 1 + 2 * i, par))
        rows.append((int(a), seq, P + 1 + i, 1, P + 2 + 2 * i, par))
    return np.array(rows, dtype=np.int32)


def row_digest(row):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(row, dtype=np.float32).tobytes()).digest(), np.uint8)


def top2_gap(row):
    """First maximum, the strict-greater runner-up, and the logit gap between them."""
    i = int(np.argmax(row))
    r = row.copy()
    r[i] = -np.inf
    j = int(np.argmax(r))
    return i, j, float(row[i] - row[j])


def file_digest(path, chunk=64 << 20, threads=8):
    """SHA-256 over the SHA-256 digests of the file's 64 MiB chunks (hashed in parallel threads)."""
    size = os.path.getsize(path)
    with open(path, "rb") as f, mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) as mm:
        view = memoryview(mm)
        try:
            with cf.ThreadPoolExecutor(threads) as ex:
                parts = list(ex.map(lambda i: hashlib.sha256(view[i * chunk:(i + 1) * chunk]).digest(),
                                    range((size + chunk - 1) // chunk)))
        finally:
            view.release()
    return hashlib.sha256(b"".join(parts)).hexdigest()


def model_config(name):
    from malkin_amd import synth
    m = MODELS[name]
    return synth.make_config(m["preset"], m["wtype"], mix=m["mix"], seed=m["seed"])


def write_model(name, directory, threads=None):
    """Writes the synthetic GGUF of case `name` into directory; returns its path."""
    from malkin_amd import synth
    path = os.path.join(directory, f"scale_{name}_{os.getpid()}.gguf")
    synth.write_gguf(path, model_config(name), threads=threads)
    return path


def model_dir(name):
    """/dev/shm when it has room for the file (with margin), else the temp directory."""
    import tempfile
    from malkin_amd import synth
    need = synth.file_bytes(model_config(name)) * 1.2
    d = "/dev/shm"
    if os.path.isdir(d):
        st = os.statvfs(d)
        if st.f_bavail * st.f_frsize > need:
            return d
    return tempfile.gettempdir()
