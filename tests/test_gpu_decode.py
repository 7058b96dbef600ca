"""The persistent decode kernel (mk_decode_layers: every layer of a one-token forward in one launch) against the
per-step launches it replaces, on synthetic Q8_0 models at the real widths of Qwen3-4B, -8B and -14B (few layers).
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
    """Each shape loaded twice: with the persistent kernel (MK_MODEL_PERSISTENT), and without."""
    d = tmp_path_factory.mktemp("decode")
    out = {}
    for i, (name, (preset, over)) in enumerate(SHAPES.items()):
        cfg = synth_lib.make_config(preset, synth_lib.Q8_0, seed=40 + i, **over)
        path = synth_lib.write_gguf(str(d / f"{name}.gguf"), cfg)
        a = mk_.Model(mk, path, N_CTX, 1, persistent=True)
        b = mk_.Model(mk, path, N_CTX, 1, persistent=False)
        print("model", name, a.cfg, "persistent", a.persistent, flush=True)
        out[name] = (a, b)
    yield out
    for a, b in out.values():
        a.close()
        b.close()


def test_plan_only_where_supported(pairs):
    for name, (a, b) in pairs.items():
        assert a.persistent == (name != "q06b"), name
        assert not b.persistent


def prompt_ids(n, vocab, seed):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.int32)


@pytest.mark.parametrize("name", ["q4b", "q8b", "q14b", "q06b"])
def test_eager_steps_match(pairs, name):
    """Prompt, then 10 one-token forwards fed with their argmax: logits and the KV rows written equal."""
    a, b = pairs[name]
    v = a.cfg["n_vocab"]
    p = prompt_ids(200, v, 7)
    la, lb = a.forward(p, 0), b.forward(p, 0)
    assert np.array_equal(bits(la), bits(lb))
    tok = int(np.argmax(la[0]))
    for step in range(10):
        pos = len(p) + step
        la = a.forward(np.array([tok], np.int32), pos)
        lb = b.forward(np.array([tok], np.int32), pos)
        print(name, "step", step, flush=True)
        assert np.array_equal(bits(la), bits(lb)), step
        tok = int(np.argmax(la[0]))
    for layer in range(a.cfg["n_layer"]):
        for pos in range(len(p), len(p) + 10):
            for k in (True, False):
                assert np.array_equal(a.kv_row(layer, 0, pos, k), b.kv_row(layer, 0, pos, k)), (layer, pos, k)


@pytest.mark.parametrize("n_prompt", [9, 600, 1100])
@pytest.mark.parametrize("use_graph", [True, False])
def test_generate_matches(pairs, n_prompt, use_graph):
    """Greedy generation (device argmax feeding the next step): identical streams with the key count spanning the
    kernel's short, medium and long attention forms."""
    a, b = pairs["q4b"]
    p = prompt_ids(n_prompt, a.cfg["n_vocab"], n_prompt)
    print("generate", n_prompt, use_graph, flush=True)
    ta, sa = a.generate(p, 40, use_graph=use_graph)
    tb, sb = b.generate(p, 40, use_graph=use_graph)
    assert list(ta) == list(tb)
    assert sa["decode_forwards"] == 39
    for layer in (0, a.cfg["n_layer"] - 1):
        for pos in (n_prompt, n_prompt + 38):
            assert np.array_equal(a.kv_row(layer, 0, pos, True), b.kv_row(layer, 0, pos, True)), (layer, pos)
            assert np.array_equal(a.kv_row(layer, 0, pos, False), b.kv_row(layer, 0, pos, False)), (layer, pos)


@pytest.mark.parametrize("name", ["q8b", "q14b"])
def test_generate_matches_wide(pairs, name):
    a, b = pairs[name]
    p = prompt_ids(300, a.cfg["n_vocab"], 11)
    ta, _ = a.generate(p, 32)
    tb, _ = b.generate(p, 32)
    assert list(ta) == list(tb)
