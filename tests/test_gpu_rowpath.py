"""The row path on the device (mk_matmul_rows; the reference's vec_dot / matmul, quant.cpp:171-191, 330-351): every
weight type it takes (F32, F16, BF16; Q8_0, Q4_K, Q5_K, Q6_K as under MALKIN_NO_PACK) bit for bit against the CPU
oracle (which test_oracle.py pins to the compiled reference), with k % 16 tails, an odd last Q8_0 block, token counts
across the kernel's 8-token tiles and row counts across its 16-row workgroups; the embedding lookup of the new
types; and whole models on the row path (F16 and BF16 weights, Q8_0 and Q4_K_M opened with MK_MODEL_NO_PACK)
against the reference's logits and greedy streams."""
import ctypes

import numpy as np
import pytest

import malkin_amd as mk_
from oracle import bind

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def row_weights(rng, t, rows, k):
    import make_golden
    if t == bind.F32:
        return rng.standard_normal((rows, k)).astype(np.float32).view(np.uint8).reshape(rows, -1)
    if t == bind.F16:
        return rng.standard_normal((rows, k)).astype(np.float16).view(np.uint8).reshape(rows, -1)
    if t == bind.BF16:
        h = (rng.standard_normal((rows, k)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        return h.view(np.uint8).reshape(rows, -1)
    return make_golden.random_rows(rng, t, rows, k)


CASES = [(t, k) for t in (bind.F32, bind.F16, bind.BF16) for k in (40, 512, 4096)] + \
    [(bind.Q8_0, k) for k in (544, 4096)] + [(t, k) for t in (bind.Q4_K, bind.Q5_K, bind.Q6_K) for k in (512, 4096)]


@pytest.mark.parametrize("t,k", CASES)
@pytest.mark.parametrize("n", [1, 3, 17])
def test_matmul_rows_vs_oracle(mk, oracle, t, k, n):
    rng = np.random.default_rng(t * 1009 + k + n)
    rows = 40  # two and a half 16-row workgroups
    w = row_weights(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    x[:, ::97] *= 50
    xq = oracle.quantize_row_q8(x) if k % 32 == 0 else None
    exp = oracle.matmul_rows(t, w, rows, k, x=x, xq=xq, n=n)
    dw, dx = mk.to_device(w), mk.to_device(x)
    dq = mk.to_device(xq) if xq is not None else None
    y0 = rng.standard_normal((n, rows)).astype(np.float32)
    for acc in (0, 1):
        dy = mk.to_device(y0)
        print("rows", t, k, n, "accumulate", acc, flush=True)
        mk_.check(mk_.load().mk_matmul_rows(mk.h, t, dw.ptr, w.shape[1], rows, k, dx.ptr, k,
                                            dq.ptr if dq is not None else None, n, dy.ptr, rows, acc))
        got = dy.download(np.float32).reshape(n, rows)
        want = (y0 + exp) if acc else exp
        assert np.array_equal(bits(got), bits(want)), (t, k, n, acc, np.abs(got - want).max())
        dy.free()


@pytest.mark.parametrize("t", [bind.F16, bind.BF16, bind.Q5_K])
def test_dequantize_rows_new_types(mk, oracle, t):
    rng = np.random.default_rng(t)
    k = 512
    w = row_weights(rng, t, 10, k)
    ids = np.array([3, 0, 9, 3], np.int32)
    dw, di = mk.to_device(w), mk.to_device(ids)
    out = mk.alloc(len(ids) * k * 4)
    mk_.check(mk_.load().mk_dequantize_rows(mk.h, t, dw.ptr, w.shape[1], di.ptr, len(ids), k, out.ptr))
    exp = np.stack([oracle.dequantize_row(t, w[i], k) for i in ids])
    assert np.array_equal(bits(out.download(np.float32).reshape(len(ids), k)), bits(exp))


ROW_MODELS = ["tiny-f16", "tiny-bf16", "tiny-nopack", "tiny-q4km-nopack"]


@pytest.fixture(scope="module")
def row_models(mk, model_files):
    import make_golden
    ms = {n: mk_.Model(mk, model_files[n], 256, 2, no_pack=make_golden.MODEL_CFGS[n].get("no_pack", False))
          for n in ROW_MODELS}
    yield ms
    for m in ms.values():
        m.close()


@pytest.mark.parametrize("name", ROW_MODELS)
def test_row_path_model_golden(row_models, golden, name):
    g = golden("models.npz")
    m = row_models[name]
    print("model", name, flush=True)
    logits = m.forward(g[f"{name}_prompt"], 0, all_logits=True)
    assert np.array_equal(bits(logits), bits(g[f"{name}_prompt_logits"])), name
    toks, last = [], logits[-1]
    for step in range(16):
        t = int(np.argmax(last))
        toks.append(t)
        last = m.forward(np.array([t], np.int32), 24 + step)[0]
    assert toks == list(g[f"{name}_greedy"])
    out, _ = m.generate(g[f"{name}_prompt"], 16, seq=1)
    assert list(out) == list(g[f"{name}_greedy"])
    batch = g[f"{name}_tree_batch"].astype(np.int32).view(mk_.BATCH_TOKEN).reshape(-1)
    assert np.array_equal(bits(m.forward_batch(batch)), bits(g[f"{name}_tree_logits"])), name


@pytest.mark.parametrize("t", [bind.Q4_K, bind.Q5_K])
@pytest.mark.parametrize("n", [1, 5, 17, 40])
def test_matmul_gguf_panel_arithmetic(mk, oracle, t, n):
    """mk_matmul_gguf: the Q4_K / Q5_K panel arithmetic over GGUF rows, against the oracle's panel restatement (and,
    for Q4_K, against the packed kernels of mk_matmul)."""
    import make_golden
    rng = np.random.default_rng(t * 31 + n)
    rows, k = 72, 1024
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    exp = oracle.matmul(t, w, rows, k, xq.reshape(-1))
    dw, dq, dy = mk.to_device(w), mk.to_device(xq), mk.alloc(n * rows * 4)
    print("gguf panel", t, n, flush=True)
    mk_.check(mk_.load().mk_matmul_gguf(mk.h, t, dw.ptr, w.shape[1], rows, k, dq.ptr, n, dy.ptr, rows, 0))
    got = dy.download(np.float32).reshape(n, rows)
    assert np.array_equal(bits(got), bits(exp)), np.abs(got - exp).max()
    if t == bind.Q4_K:
        pk = mk.alloc(mk_.load().mk_packed_bytes(t, rows, k))
        mk_.check(mk_.load().mk_pack_weight(mk.h, t, dw.ptr, w.shape[1], rows, k, pk.ptr))
        wt = mk_.MkWeight(t, 1, rows, k, pk.p)
        mk_.check(mk_.load().mk_matmul(mk.h, ctypes.byref(wt), dq.ptr, n, dy.ptr, rows, 0))
        assert np.array_equal(bits(dy.download(np.float32).reshape(n, rows)), bits(exp))


def test_matmul_gguf_q5k_golden(mk, golden):
    """The reference's own Q5_K panel outputs (gemm.npz, written by oracle/_ref, compact and wide panels)."""
    g = golden("gemm.npz")
    ci = next(i for i in range(8) if f"c{i}_type" in g.files and int(g[f"c{i}_type"]) == bind.Q5_K)
    w = g[f"c{ci}_w"]
    rows, k = w.shape[0], w.shape[1] // 176 * 256
    for key in g.files:
        if not (key.startswith(f"c{ci}_n") and key.endswith("_xq")):
            continue
        n = int(key[len(f"c{ci}_n"):-3])
        xq = g[key]
        dw, dq, dy = mk.to_device(w), mk.to_device(xq), mk.alloc(n * rows * 4)
        mk_.check(mk_.load().mk_matmul_gguf(mk.h, bind.Q5_K, dw.ptr, w.shape[1], rows, k, dq.ptr, n, dy.ptr, rows, 0))
        got = dy.download(np.float32).reshape(n, rows)
        for ref_key in (f"c{ci}_n{n}_y", f"c{ci}_n{n}_y_compact"):
            assert np.array_equal(bits(got), bits(g[ref_key])), ref_key


def test_q5k_model_golden(mk, model_files, golden):
    g = golden("models.npz")
    name = "tiny-q5k"
    m = mk_.Model(mk, model_files[name], 256, 2)
    try:
        logits = m.forward(g[f"{name}_prompt"], 0, all_logits=True)
        assert np.array_equal(bits(logits), bits(g[f"{name}_prompt_logits"]))
        last = logits[-1]
        for step in range(16):  # the stream on sequence 0 (the tree batch below continues it)
            t = int(np.argmax(last))
            assert t == g[f"{name}_greedy"][step]
            last = m.forward(np.array([t], np.int32), 24 + step)[0]
        out, _ = m.generate(g[f"{name}_prompt"], 16, seq=1)
        assert list(out) == list(g[f"{name}_greedy"])
        batch = g[f"{name}_tree_batch"].astype(np.int32).view(mk_.BATCH_TOKEN).reshape(-1)
        assert np.array_equal(bits(m.forward_batch(batch)), bits(g[f"{name}_tree_logits"]))
    finally:
        m.close()
