"""The persistent decode kernel (mk_decode_layers: every layer of a one-token forward in one launch) and the fused
attention + attn_output launch (mk_decode_attn_wo) against the per-step launches they replace, on synthetic Q8_0
models at the real widths of Qwen3-4B, -8B and -14B (few layers).
The per-step path is pinned to the reference elsewhere (test_gpu_model.py, test_gpu_scale.py); here every logit and
every KV cache byte of the persistent path must equal it bit for bit, over short, medium and long rows (the kernel's
attention takes 2, 4 or 8 staging slots), eager forwards and replayed graphs."""
import numpy as np
import pytest

import malkin_amd as mk_

pytestmark = pytest.mark.gpu

N_CTX = 2048

# name: (preset, overrides). 0.6B's 1024-wide rows are too short for the kernel (no plan: per-step launches).
SHAPES = {
    "q4b": ("qwen3-4b", dict(n_layer=3, n_vocab=4096)),
    "q8b": ("qwen3-8b", dict(n_layer=2, n_vocab=4096)),
    "q14b": ("qwen3-14b", dict(n_layer=2, n_vocab=4096)),
    "q06b": ("qwen3-0.6b", dict(n_layer=2, n_vocab=4096)),
}


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def pairs(mk, synth_lib, tmp_path_factory):
    """Each shape loaded three times: with the persistent kernel (MK_MODEL_PERSISTENT), with per-step launches, and
    with the fused attention + attn_output launch (MK_MODEL_FUSED_ATTN)."""
    d = tmp_path_factory.mktemp("decode")
    out = {}
    for i, (name, (preset, over)) in enumerate(SHAPES.items()):
        cfg = synth_lib.make_config(preset, synth_lib.Q8_0, seed=40 + i, **over)
        path = synth_lib.write_gguf(str(d / f"{name}.gguf"), cfg)
        a = mk_.Model(mk, path, N_CTX, 1, persistent=True)
        b = mk_.Model(mk, path, N_CTX, 1, persistent=False)
        c = mk_.Model(mk, path, N_CTX, 1, fused_attn=True)
        print("model", name, a.cfg, "persistent", a.persistent, "fused", c.fused_attn, flush=True)
        out[name] = (a, b, c)
    yield out
    for ms in out.values():
        for m in ms:
            m.close()


def test_plan_only_where_supported(pairs):
    for name, (a, b, c) in pairs.items():
        assert a.persistent == (name != "q06b"), name
        assert not b.persistent and not b.fused_attn
        assert c.fused_attn == (name != "q06b") and not c.persistent, name


def prompt_ids(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


@pytest.mark.parametrize("name", ["q4b", "q8b", "q14b", "q06b"])
def test_eager_steps_match(pairs, name):
    """Prompt, then 10 one-token forwards fed with their argmax: logits and the KV rows written equal."""
    a, b, c = pairs[name]
    v = a.cfg["n_vocab"]
    p = prompt_ids(200, v, 7)
    la, lb, lc = a.forward(p, 0), b.forward(p, 0), c.forward(p, 0)
    assert np.array_equal(bits(la), bits(lb)) and np.array_equal(bits(lc), bits(lb))
    tok = int(np.argmax(la[0]))
    for step in range(10):
        pos = len(p) + step
        la = a.forward(np.array([tok], np.int32), pos)
        lb = b.forward(np.array([tok], np.int32), pos)
        lc = c.forward(np.array([tok], np.int32), pos)
        print(name, "step", step, flush=True)
        assert np.array_equal(bits(la), bits(lb)), step
        assert np.array_equal(bits(lc), bits(lb)), ("fused", step)
        tok = int(np.argmax(la[0]))
    for layer in range(a.cfg["n_layer"]):
        for pos in range(len(p), len(p) + 10):
            for k in (True, False):
                assert np.array_equal(a.kv_row(layer, 0, pos, k), b.kv_row(layer, 0, pos, k)), (layer, pos, k)
                assert np.array_equal(c.kv_row(layer, 0, pos, k), b.kv_row(layer, 0, pos, k)), ("fused", layer, pos)


@pytest.mark.parametrize("n_prompt", [9, 600, 1100])
@pytest.mark.parametrize("use_graph", [True, False])
def test_generate_matches(pairs, n_prompt, use_graph):
    """Greedy generation (device argmax feeding the next step): identical streams with the key count spanning the
    kernel's short, medium and long attention forms."""
    a, b, c = pairs["q4b"]
    p = prompt_ids(n_prompt, a.cfg["n_vocab"], n_prompt)
    print("generate", n_prompt, use_graph, flush=True)
    ta, sa = a.generate(p, 40, use_graph=use_graph)
    tb, sb = b.generate(p, 40, use_graph=use_graph)
    tc, sc = c.generate(p, 40, use_graph=use_graph)
    assert list(ta) == list(tb) and list(tc) == list(tb)
    assert sa["decode_forwards"] == 39
    for layer in (0, a.cfg["n_layer"] - 1):
        for pos in (n_prompt, n_prompt + 38):
            assert np.array_equal(a.kv_row(layer, 0, pos, True), b.kv_row(layer, 0, pos, True)), (layer, pos)
            assert np.array_equal(a.kv_row(layer, 0, pos, False), b.kv_row(layer, 0, pos, False)), (layer, pos)


@pytest.mark.parametrize("name", ["q8b", "q14b"])
def test_generate_matches_wide(pairs, name):
    a, b, c = pairs[name]
    p = prompt_ids(300, a.cfg["n_vocab"], 11)
    ta, _ = a.generate(p, 32)
    tb, _ = b.generate(p, 32)
    tc, _ = c.generate(p, 32)
    assert list(ta) == list(tb) and list(tc) == list(tb)
