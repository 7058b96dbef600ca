"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it:

  * against the golden vectors written by the reference's own compiled hot path (tests/golden/*.npz), bit for bit;
  * against the compiled reference directly on fresh random inputs, where it is built here (oracle/_ref);
  * against what the mathematics fixes, independently of the reference: closed forms, brute-force integer dots,
    float64 references with the reference's own tolerances (test_quant.cpp), exact invariants.
"""
import math

import numpy as np
import pytest

from oracle import bind


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def fma32(a, b, c):
    """Exact fp32 fused multiply-add (one rounding, to nearest even), computed with rationals."""
    from fractions import Fraction
    x = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    if x == 0:
        return np.float32(0.0)
    sign, x = (-1 if x < 0 else 1), abs(x)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    while Fraction(2) ** e > x:
        e -= 1
    while Fraction(2) ** (e + 1) <= x:
        e += 1
    q = max(e, -126) - 23  # unit in the last place
    m = x / Fraction(2) ** q
    r = m.numerator // m.denominator
    rem = m - r
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and r % 2 == 1):
        r += 1
    return np.float32(sign * float(r * Fraction(2) ** q))


# ---------------------------------------------------------------- golden vectors


def test_quantize_q8_golden(oracle, golden):
    g = golden("quant.npz")
    got = oracle.quantize_row_q8(g["x"]).view(np.uint8)
    assert np.array_equal(got.reshape(-1), g["q8"].reshape(-1))


def test_quantize_i8_golden(oracle, golden):
    g = golden("quant.npz")
    for x, q, d in zip(g["xi"], g["qi"], g["di"]):
        gq, gd = oracle.quantize_i8(x)
        assert np.array_equal(gq, q) and bits(np.float32(gd)) == bits(d)


def test_silu_dot_golden(oracle, golden):
    g = golden("quant.npz")
    assert np.array_equal(bits(oracle.silu_mul(g["g"], g["u"])), bits(g["silu"]))
    for w, d in zip(g["w"], g["dots"]):
        assert bits(oracle.dot_f32(w, w)) == bits(d)


def test_gemm_golden(oracle, golden):
    g = golden("gemm.npz")
    cases = sorted({k.split("_")[0] for k in g.files})
    checked = 0
    for c in cases:
        t = int(g[f"{c}_type"])
        w = g[f"{c}_w"]
        rows = w.shape[0]
        k = w.shape[1] // (34 if t == bind.Q8_0 else {12: 144, 13: 176, 14: 210}[t]) * (32 if t == bind.Q8_0 else 256)
        for key in g.files:
            if key.startswith(c + "_n") and key.endswith("_xq"):
                n = key[len(c) + 2:-3]
                xq = g[key].view(bind.BLOCK_Q8)
                y = oracle.matmul(t, w, rows, k, xq, wide=True)
                assert np.array_equal(bits(y), bits(g[f"{c}_n{n}_y"])), (c, n, "wide")
                yc = oracle.matmul(t, w, rows, k, xq, wide=False)
                assert np.array_equal(bits(yc), bits(g[f"{c}_n{n}_y_compact"])), (c, n, "compact")
                checked += 1
    assert checked >= 12


def test_attention_golden(oracle, golden):
    g = golden("attention.npz")
    for i in range(int(g["count"])):
        G, D, n, ne, stride = (int(v) for v in g[f"a{i}_meta"])
        extra = g[f"a{i}_extra"] if ne else None
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        out = oracle.attend_gqa(g[f"a{i}_q"], G, D, g[f"a{i}_k"], g[f"a{i}_v"], stride, D + 4, n, scale, extra)
        assert np.array_equal(bits(out), bits(g[f"a{i}_out"])), (G, D, n)


def test_model_golden(oracle, golden, model_files):
    import hashlib
    import make_golden
    g = golden("models.npz")
    for name, path in model_files.items():
        with open(path, "rb") as f:
            assert hashlib.sha256(f.read()).digest() == bytes(g[f"{name}_sha256"]), f"synthetic {name} drifted"
        m = oracle.model(path, 256, 2, no_pack=make_golden.MODEL_CFGS[name].get("no_pack", False))
        logits = m.forward(g[f"{name}_prompt"], 0, all_logits=True)
        assert np.array_equal(bits(logits), bits(g[f"{name}_prompt_logits"])), name
        toks, last = [], logits[-1]
        for step in range(16):
            t = oracle.argmax(last)
            toks.append(t)
            last = m.forward(np.array([t], np.int32), 24 + step)[0]
        assert toks == list(g[f"{name}_greedy"]), name
        batch = g[f"{name}_tree_batch"].astype(np.int32).view(bind.BATCH_TOKEN).reshape(-1)
        tl = m.forward_batch(batch)
        assert np.array_equal(bits(tl), bits(g[f"{name}_tree_logits"])), name
        m.close()


# ---------------------------------------------------------------- against the compiled reference, fresh inputs


def test_against_reference_random(oracle, ref):
    rng = np.random.default_rng(1234)
    for _ in range(20):
        x = (rng.standard_normal((4, 512)) * rng.uniform(0.01, 100)).astype(np.float32)
        assert np.array_equal(oracle.quantize_row_q8(x).view(np.uint8), ref.quantize_row_q8(x).view(np.uint8))
        g = rng.uniform(-40, 40, 1024).astype(np.float32)
        u = rng.uniform(-2, 2, 1024).astype(np.float32)
        assert np.array_equal(bits(oracle.silu_mul(g, u)), bits(ref.silu_mul(g, u)))
        k = int(rng.choice([16, 100, 128, 4096]))
        w = rng.standard_normal(k).astype(np.float32)
        assert bits(oracle.dot_f32(w, w)) == bits(ref.dot_f32(w, w))


def _row_weights(rng, t, rows, k):
    import make_golden
    if t == bind.F32:
        return rng.standard_normal((rows, k)).astype(np.float32).view(np.uint8).reshape(rows, -1)
    if t == bind.F16:
        return rng.standard_normal((rows, k)).astype(np.float16).view(np.uint8).reshape(rows, -1)
    if t == bind.BF16:
        h = (rng.standard_normal((rows, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        return h.view(np.uint8).reshape(rows, -1)
    return make_golden.random_rows(rng, t, rows, k)


ROW_CASES = [(t, k) for t in (bind.F32, bind.F16, bind.BF16) for k in (40, 512, 4096)] + \
    [(bind.Q8_0, k) for k in (512, 544, 4096)] + [(t, k) for t in (bind.Q4_K, bind.Q5_K, bind.Q6_K) for k in (512, 4096)]


@pytest.mark.parametrize("t,k", ROW_CASES)
def test_row_path_against_reference(oracle, ref, t, k):
    """The row path (vec_dot, quant.cpp:171-191): F types with a k % 16 tail, Q8_0 with an odd last block."""
    rng = np.random.default_rng(t * 10007 + k)
    w = _row_weights(rng, t, 6, k)
    x = rng.uniform(-2, 2, (3, k)).astype(np.float32)
    x[:, ::97] *= 50
    xq = ref.quantize_row_q8(x) if k % 32 == 0 else None
    yo = oracle.matmul_rows(t, w, 6, k, x=x, xq=xq, n=3)
    yr = ref.matmul_rows(t, w, 6, k, x=x, xq=xq, n=3)
    assert np.array_equal(bits(yo), bits(yr))


@pytest.mark.parametrize("t,k", [(t, k) for t, k in ROW_CASES if k >= 512])
def test_row_path_vs_float64(oracle, t, k):
    """Independent of the reference: every row-path output is the dot of the dequantized operands (float64) within
    the reference's own |d|/rms < 1e-5 (test_quant.cpp:250-256); the F types against the fp32 activations."""
    rng = np.random.default_rng(t + k)
    w = _row_weights(rng, t, 8, k)
    x = rng.uniform(-2, 2, (2, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    y = oracle.matmul_rows(t, w, 8, k, x=x, xq=xq, n=2)
    wd = np.stack([oracle.dequantize_row(t, w[r], k) for r in range(8)]).astype(np.float64)
    if t in (bind.F32, bind.F16, bind.BF16):
        xd = x.astype(np.float64)
    else:  # the BlockQ8 values d * q, exactly
        xd = (xq["d"].astype(np.float64)[..., None] * xq["qs"].astype(np.float64)).reshape(2, k)
    exp = xd @ wd.T
    err = np.abs(y - exp).max() / np.sqrt((exp ** 2).mean())
    assert err < 1e-5, err


def test_model_against_reference(oracle, ref, model_files):
    """Batched multi-sequence and tree-verify forwards, plus move_kv, on fresh inputs."""
    rng = np.random.default_rng(99)
    for name in ("tiny", "tiny-q6k"):
        om = oracle.model(model_files[name], 128, 3)
        rm = ref.model(model_files[name], 128, 3)
        V = om.cfg["n_vocab"]
        for s in range(3):
            p = rng.integers(0, V, 20 + 3 * s).astype(np.int32)
            assert np.array_equal(bits(om.forward(p, 0, seq=s)), bits(rm.forward(p, 0, seq=s)))
        # one batch: decode token of seq 0, tree of seq 1, chunk of seq 2
        b = [(5, 0, 20, 1, -1, -1), (7, 1, 23, 1, -1, -1), (9, 1, 24, 1, 24, 1), (11, 1, 24, 1, 25, 1),
             (13, 1, 25, 1, 26, 2)] + [(int(t), 2, 26 + j, int(j == 3), -1, -1) for j, t in
                                       enumerate(rng.integers(0, V, 4))]
        batch = np.array(b, dtype=bind.BATCH_TOKEN)
        assert np.array_equal(bits(om.forward_batch(batch)), bits(rm.forward_batch(batch)))
        om.move_kv(26, 24, 1)
        rm.move_kv(26, 24, 1)
        nxt = np.array([3, 4], np.int32)
        assert np.array_equal(bits(om.forward(nxt, 25, seq=1)), bits(rm.forward(nxt, 25, seq=1)))
        # tree through the other forward entry point (model.cpp:249-278)
        par = np.array([-1, 0, 0, 1], np.int32)
        tl = rng.integers(0, V, 4).astype(np.int32)
        assert np.array_equal(bits(om.forward(tl, 27, True, par, 1)), bits(rm.forward(tl, 27, True, par, 1)))
        for msg_batch in ([(1, 5, 0, 1, -1, -1)], [(1, 0, 0, 1, -1, -1), (2, 1, 1, 1, 1, 0)]):
            bb = np.array(msg_batch, dtype=bind.BATCH_TOKEN)
            with pytest.raises(RuntimeError) as eo:
                om.forward_batch(bb)
            with pytest.raises(RuntimeError) as er:
                rm.forward_batch(bb)
            assert str(eo.value) == str(er.value)


# ---------------------------------------------------------------- mathematics, independent of the reference


def test_quantize_q8_closed_form(oracle):
    """check_q8_sums (test_quant.cpp:92-108) and the closed form of kernels_avx512.cpp:66-80."""
    rng = np.random.default_rng(5)
    x = rng.uniform(-3, 3, (16, 256)).astype(np.float32)
    x[0, :32] = 0
    q = oracle.quantize_row_q8(x).reshape(-1)
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / d, np.float32(0)).astype(np.float32)
    qs = np.rint((xb * idv[:, None]).astype(np.float32)).astype(np.int32)
    assert np.array_equal(q["d"], d)
    assert np.array_equal(q["qs"].astype(np.int32), np.clip(qs, -128, 127))
    assert np.array_equal(q["s"][:, 0], qs[:, :16].sum(1)) and np.array_equal(q["s"][:, 1], qs[:, 16:].sum(1))
    assert np.abs(q["qs"]).max() == 127


def test_exp_polynomial_accuracy(oracle):
    """exp512 is a degree-6 Taylor after Cody-Waite reduction: relative error ~1e-7 over the softmax range; a wrong
    constant or a dropped term shows up far above that."""
    xs = np.linspace(-87, 0, 20001, dtype=np.float32)
    worst = max(abs(float(oracle.exp(x)) / math.exp(float(x)) - 1) for x in xs[::7])
    assert worst < 3e-7
    assert float(oracle.exp(np.float32(-200))) == pytest.approx(math.exp(-87), rel=1e-6)  # clamped at -87
    assert math.isinf(float(oracle.exp(np.float32(200))))


def test_reduce16_tree(oracle):
    import ctypes
    v = np.array([1e8, 1, -1e8, 1] + [0] * 12, dtype=np.float32)
    # halving tree: (v0 + v8) + (v4 + v12) ... ; 1e8 + 0 and -1e8 + 0 cancel in the last step, so both 1s survive
    got = oracle.lib.or_reduce16(v.ctypes.data_as(ctypes.c_void_p))
    assert got == 2.0
    w = np.array([1e8, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 0], dtype=np.float32)
    assert oracle.lib.or_reduce16(w.ctypes.data_as(ctypes.c_void_p)) == np.float32(1e8) + np.float32(1)


@pytest.mark.parametrize("t,k", [(bind.Q8_0, 2560), (bind.Q8_0, 96), (bind.Q4_K, 2560), (bind.Q5_K, 2560),
                                 (bind.Q6_K, 2560)])
def test_gemm_vs_float64(oracle, t, k):
    """check / check_gemm (test_quant.cpp:61-90, 213-262): panel result vs a float64 dot of the dequantized operands,
    rel < 1e-5 of sum |w x|; and the per-block integer dots reproduced exactly by brute force (Q8_0)."""
    rng = np.random.default_rng(t * 1000 + k)
    import make_golden
    rows = 8
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (3, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    y = oracle.matmul(t, w, rows, k, xq.reshape(-1))
    xr = (xq["d"][..., None] * xq["qs"].astype(np.float32)).reshape(3, k).astype(np.float64)
    for r in range(rows):
        wr = oracle.dequantize_row(t, w[r], k).astype(np.float64)
        ref = xr @ wr
        mag = np.abs(xr * wr).sum(1)
        assert np.all(np.abs(y[:, r] - ref) / (mag + 1e-6) < 1e-5)
    if t == bind.Q8_0:  # exact int dots: reconstruct y with the reference's epilogue from brute-force integers
        for r in range(rows):
            blk = w[r].reshape(-1, 34)
            dw = blk[:, :2].copy().view(np.float16).astype(np.float32).ravel()
            qw = blk[:, 2:].view(np.int8).astype(np.int64)
            for tt in range(3):
                ai = (qw * xq["qs"][tt].astype(np.int64)).sum(1)
                acc = np.float32(0)
                for b in range(len(ai)):
                    p = np.float32(dw[b] * xq["d"][tt][b])
                    acc = fma32(np.float32(ai[b]), p, acc)
                assert bits(acc) == bits(y[tt, r])


def test_attention_vs_float64(oracle):
    """check_attention (test_quant.cpp:137-176): vs a double-precision reference, abs error < 1e-4."""
    import make_golden
    rng = np.random.default_rng(7)
    for G in (1, 2, 4):
        for D in (64, 80, 128):
            for n in (1, 7, 300):
                ne = 3 if n > 1 else 0
                stride = D + 16
                k = make_golden.fill_kv(rng, n + 5, stride, D)
                v = make_golden.fill_kv(rng, n + 5, stride, D)
                q = rng.uniform(-3, 3, G * D).astype(np.float32)
                extra = np.array([n + 4, n + 1, n + 2][:ne], np.int32)
                scale = np.float32(1) / np.sqrt(np.float32(D))
                out = oracle.attend_gqa(q, G, D, k, v, stride, D + 4, n, scale, extra if ne else None)
                rows = list(range(n)) + list(extra)
                ks = np.array([k[r, D + 4:D + 8].view(np.float32)[0] for r in rows], np.float64)
                vs = np.array([v[r, D + 4:D + 8].view(np.float32)[0] for r in rows], np.float64)
                K = k[rows, :D].astype(np.float64)
                V = v[rows, :D].astype(np.float64)
                for h in range(G):
                    s = K @ q[h * D:(h + 1) * D].astype(np.float64) * ks * float(scale)
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    o = (p * vs) @ V
                    assert np.abs(out[h * D:(h + 1) * D] - o).max() < 1e-4


def test_silu_vs_float64(oracle):
    """test_quant.cpp:200-208: <= 1e-5 (1 + |ref|), including x = -200."""
    rng = np.random.default_rng(3)
    g = (30 * rng.uniform(-1, 1, 64)).astype(np.float32)
    u = rng.uniform(-1, 1, 64).astype(np.float32)
    g[0] = -200
    got = oracle.silu_mul(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.all(np.abs(got - ref) <= 1e-5 * (1 + np.abs(ref)))


def test_argmax_top2_ties(oracle):
    l = np.array([3, 5, 5, 1, 5, 4], np.float32)
    assert oracle.argmax(l) == 1  # first maximum (std::max_element)
    assert oracle.top2(l) == (1, 2)
    assert oracle.top2(np.array([5, 5], np.float32)) == (0, 1)
    assert oracle.top2(np.array([4, 6, 5, 6], np.float32)) == (1, 3)
    rng = np.random.default_rng(0)
    for _ in range(200):
        l = rng.integers(0, 6, 50).astype(np.float32)
        a, b = oracle.top2(l)
        assert a == int(np.argmax(l))
        rest = l.copy()
        rest[a] = -np.inf
        assert b == int(np.argmax(rest))


def test_dequantize_closed_forms(oracle):
    rng = np.random.default_rng(8)
    import make_golden
    w = make_golden.random_rows(rng, bind.Q8_0, 1, 64)[0]
    y = oracle.dequantize_row(bind.Q8_0, w, 64)
    blk = w.reshape(2, 34)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(y.reshape(2, 32), d * blk[:, 2:].view(np.int8).astype(np.float32))
    for h in (0, 0x3C00, 0x0001, 0x03FF, 0x7BFF, 0x8400, 0xC000):  # f16 incl. subnormals
        assert oracle.fp16_to_fp32(h) == np.uint16(h).view(np.float16).astype(np.float32)
        assert oracle.fp32_to_fp16(oracle.fp16_to_fp32(h)) == h
    for f in (0.1, 1e-5, 65504.0, 1e-8, 3.14159):
        assert oracle.fp32_to_fp16(f) == np.float16(np.float32(f)).view(np.uint16)
