"""Writes the golden vectors under tests/golden/ by running the reference's own hot path, compiled from its sources
(oracle/_ref/libmalkin_ref.so, built by oracle/Makefile where /root/reference exists), on seeded inputs.

    python tests/golden/make_golden.py

Fixtures are data only (inputs and the reference's outputs), saved with numpy (no pickles). The synthetic model
files are not stored: they are regenerated bit-identically by malkin_amd/synth from the recorded config, and their
SHA-256 is stored alongside to prove it.
"""
import hashlib
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from malkin_amd import synth  # noqa: E402
from oracle import bind  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def sha256(path):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for chunk in iter(lambda: f.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def random_rows(rng, t, rows, k):
    """Random blocks with sane half scales (the scheme of test_quant.cpp:22-59)."""
    rb = bind.row_size(t, k)
    data = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
    def put_half(col_bytes, vals):
        return np.asarray(vals, dtype=np.float64).astype(np.float16).view(np.uint16)
    if t == bind.Q8_0:
        for b in range(k // 32):
            h = put_half(None, rng.uniform(0.001, 0.02, size=rows))
            data[:, 34 * b] = h & 0xFF
            data[:, 34 * b + 1] = h >> 8
    elif t in (bind.Q4_K, bind.Q5_K):
        bs = 144 if t == bind.Q4_K else 176
        for b in range(k // 256):
            for off in (0, 2):
                h = put_half(None, rng.uniform(0.001, 0.02, size=rows))
                data[:, bs * b + off] = h & 0xFF
                data[:, bs * b + off + 1] = h >> 8
    elif t == bind.Q6_K:
        for b in range(k // 256):
            h = put_half(None, rng.uniform(0.001, 0.02, size=rows))
            data[:, 210 * b + 208] = h & 0xFF
            data[:, 210 * b + 209] = h >> 8
    return data


def fill_kv(rng, rows, stride, D):
    """int8 KV rows of `stride` bytes: D values, a float scale at D + 4 (test_quant.cpp:110-119)."""
    kv = rng.integers(-127, 128, size=(rows, stride), dtype=np.int64).astype(np.int8)
    s = rng.uniform(0.005, 0.03, size=rows).astype(np.float32)
    kv[:, D + 4:D + 8] = s.view(np.int8).reshape(rows, 4)
    return kv


def gen_quant(ref, rng):
    x = rng.uniform(-3, 3, size=(6, 256)).astype(np.float32)
    x[1, :32] = 0.0                      # all-zero block: d = 0
    x[2] *= 100.0                        # large values
    x[3, ::97] *= 100.0                  # outlier channels
    x[4, :32] = np.float32(1e-30)        # tiny block
    x[5] = np.round(x[5] * 4) / 4        # exact ties after scaling
    q8 = ref.quantize_row_q8(x)
    xi = rng.normal(0, 1, size=(5, 128)).astype(np.float32)
    xi[0] = 0
    qi, di = [], []
    for r in xi:
        q, d = ref.quantize_i8(r)
        qi.append(q)
        di.append(d)
    g = rng.uniform(-30, 30, size=4096).astype(np.float32)
    g[0] = -200.0
    g[1] = 200.0
    g[2] = 0.0
    g[3] = -0.0
    u = rng.uniform(-1, 1, size=4096).astype(np.float32)
    silu = ref.silu_mul(g, u)
    w = rng.normal(0, 1, size=(3, 4096)).astype(np.float32)
    dots = np.array([ref.dot_f32(wi, wi) for wi in w], dtype=np.float32)
    np.savez_compressed(os.path.join(OUT, "quant.npz"), x=x, q8=q8.view(np.uint8), xi=xi, qi=np.array(qi),
                        di=np.array(di, dtype=np.float32), g=g, u=u, silu=silu, w=w, dots=dots)


def gen_gemm(ref, rng):
    out = {}
    cases = [(bind.Q8_0, 24, 512, (1, 3, 8, 17)), (bind.Q8_0, 16, 96, (1, 2)), (bind.Q4_K, 24, 512, (1, 4, 17)),
             (bind.Q5_K, 16, 512, (1, 5)), (bind.Q6_K, 24, 512, (1, 4, 17, 23))]
    for ci, (t, rows, k, ns) in enumerate(cases):
        w = random_rows(rng, t, rows, k)
        out[f"c{ci}_type"] = np.array(t)
        out[f"c{ci}_w"] = w
        for n in ns:
            x = rng.uniform(-2, 2, size=(n, k)).astype(np.float32)
            x[:, ::97] *= 100.0
            xq = ref.quantize_row_q8(x)
            out[f"c{ci}_n{n}_xq"] = xq.view(np.uint8)
            out[f"c{ci}_n{n}_y"] = ref.matmul(t, w, rows, k, xq.reshape(-1), mode=2)      # with wide panels
            out[f"c{ci}_n{n}_y_compact"] = ref.matmul(t, w, rows, k, xq.reshape(-1), mode=1)
    np.savez_compressed(os.path.join(OUT, "gemm.npz"), **out)


def gen_attention(ref, rng):
    out = {}
    i = 0
    for G in (1, 2, 4, 5):
        for D in (64, 80, 128):
            for n in (1, 7, 160):
                ne = 3 if n > 1 else 0
                stride = D + 16
                k = fill_kv(rng, n + 5, stride, D)
                v = fill_kv(rng, n + 5, stride, D)
                q = rng.uniform(-3, 3, size=G * D).astype(np.float32)
                extra = np.array([n + 4, n + 1, n + 2][:ne], dtype=np.int32)
                scale = np.float32(1.0) / np.sqrt(np.float32(D))
                o = ref.attend_gqa(q, G, D, k, v, stride, D + 4, n, scale, extra if ne else None)
                out[f"a{i}_meta"] = np.array([G, D, n, ne, stride], dtype=np.int64)
                out[f"a{i}_q"], out[f"a{i}_k"], out[f"a{i}_v"], out[f"a{i}_extra"], out[f"a{i}_out"] = q, k, v, extra, o
                i += 1
    out["count"] = np.array(i)
    np.savez_compressed(os.path.join(OUT, "attention.npz"), **out)


MODEL_CFGS = {
    "tiny": dict(preset="tiny", wtype=synth.Q8_0, seed=7),
    "tiny-tied": dict(preset="tiny-tied", wtype=synth.Q8_0, seed=11),
    "tiny-q6k": dict(preset="tiny", wtype=synth.Q6_K, seed=13),
    "tiny-q4km": dict(preset="tiny", wtype=synth.Q4_K, mix=synth.MIX_Q4_K_M, seed=17),
    # the row path (quant.cpp:171-191, 330-351): F16 / BF16 weights always, the quantized types under MALKIN_NO_PACK
    "tiny-f16": dict(preset="tiny", wtype=synth.F16, seed=19),
    "tiny-bf16": dict(preset="tiny-tied", wtype=synth.BF16, seed=23),
    "tiny-nopack": dict(preset="tiny", wtype=synth.Q8_0, seed=29, no_pack=True),
    "tiny-q4km-nopack": dict(preset="tiny", wtype=synth.Q4_K, mix=synth.MIX_Q4_K_M, seed=31, no_pack=True),
    # Q5_K: the panel arithmetic (gemm_avx512.cpp:104-155, kHigh)
    "tiny-q5k": dict(preset="tiny", wtype=synth.Q5_K, seed=37),
}


def model_path(tmp, name):
    c = MODEL_CFGS[name]
    cfg = synth.make_config(c["preset"], c["wtype"], mix=c.get("mix", 0), seed=c["seed"])
    p = os.path.join(tmp, name + ".gguf")
    synth.write_gguf(p, cfg, threads=4)
    return p


def gen_models(ref, rng):
    # one generator in MODEL_CFGS order: models appended at the end leave the earlier fixtures unchanged
    out = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name in MODEL_CFGS:
            p = model_path(tmp, name)
            out[f"{name}_sha256"] = np.frombuffer(bytes.fromhex(sha256(p)), dtype=np.uint8)
            m = ref.model(p, 256, 2, no_pack=MODEL_CFGS[name].get("no_pack", False))
            V = m.cfg["n_vocab"]
            prompt = rng.integers(0, V, size=24).astype(np.int32)
            logits = m.forward(prompt, 0, all_logits=True)
            out[f"{name}_prompt"] = prompt
            out[f"{name}_prompt_logits"] = logits
            toks, last = [], logits[-1]
            for step in range(16):  # greedy stream: argmax = first maximum (sampler.cpp:27-30)
                t = int(np.argmax(last))
                toks.append(t)
                last = m.forward(np.array([t], np.int32), 24 + step)[0]
            out[f"{name}_greedy"] = np.array(toks, dtype=np.int32)
            # Tree verify (model.cpp:280-323): next token + chain/alt pairs after the 24-token prefix of sequence 0.
            P = 24 + 16
            seq1 = rng.integers(0, V, size=10).astype(np.int32)
            b = [(int(toks[-1]), 0, P, 1, -1, -1)]
            for i in range(3):
                par = 0 if i == 0 else 2 * i - 1
                b.append((int(rng.integers(0, V)), 0, P + 1 + i, 1, P + 1 + 2 * i, par))
                b.append((int(rng.integers(0, V)), 0, P + 1 + i, 1, P + 2 + 2 * i, par))
            for j, t in enumerate(seq1):  # a prompt chunk of sequence 1 in the same batch
                b.append((int(t), 1, j, 1 if j == len(seq1) - 1 else 0, -1, -1))
            batch = np.array(b, dtype=bind.BATCH_TOKEN)
            out[f"{name}_tree_batch"] = batch.view(np.int32).reshape(len(b), 6)
            out[f"{name}_tree_logits"] = m.forward_batch(batch)
            m.close()
    np.savez_compressed(os.path.join(OUT, "models.npz"), **out)


def main():
    ref = bind.Ref()
    if not ref.cpu_ok():
        raise SystemExit("this CPU cannot run the reference's AVX-512 path")
    ref.set_threads(4)
    gen_quant(ref, np.random.default_rng(42))
    gen_gemm(ref, np.random.default_rng(43))
    gen_attention(ref, np.random.default_rng(44))
    gen_models(ref, np.random.default_rng(45))
    for f in sorted(os.listdir(OUT)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(OUT, f)))


if __name__ == "__main__":
    main()
