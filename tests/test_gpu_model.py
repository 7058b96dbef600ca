"""Model-level parity on the device: the full Qwen3 forward (prefill, decode, batched multi-sequence and tree-verify
batches, move_kv, KV cache rows) and greedy token streams, bit-identical to the golden vectors of the reference and
to the CPU oracle on fresh inputs. Error behaviour matches the reference's runtime_error texts."""
import numpy as np
import pytest

import malkin_amd as mk_
from oracle import bind

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.fixture(scope="module")
def models(mk, model_files):
    ms = {name: mk_.Model(mk, path, 256, 2) for name, path in model_files.items()}
    yield ms
    for m in ms.values():
        m.close()


@pytest.mark.parametrize("name", ["tiny", "tiny-tied", "tiny-q6k", "tiny-q4km"])
def test_prompt_logits_golden(models, golden, name):
    g = golden("models.npz")
    m = models[name]
    print("model", name, m.cfg, flush=True)
    logits = m.forward(g[f"{name}_prompt"], 0, all_logits=True)
    assert np.array_equal(bits(logits), bits(g[f"{name}_prompt_logits"]))


@pytest.mark.parametrize("name", ["tiny", "tiny-tied", "tiny-q6k", "tiny-q4km"])
def test_greedy_stream_golden(models, golden, name):
    g = golden("models.npz")
    m = models[name]
    m.forward(g[f"{name}_prompt"], 0, all_logits=True)
    toks, t1 = [], None
    b = mk_.batch([(0, 0, 0, 1)])
    logits = m.forward(g[f"{name}_prompt"], 0)
    last = logits[0]
    for step in range(16):
        t = int(np.argmax(last))
        toks.append(t)
        last = m.forward(np.array([t], np.int32), 24 + step)[0]
    assert toks == list(g[f"{name}_greedy"])
    # device-side argmax + graph-replayed decode loop: the same stream
    for use_graph in (False, True):
        out, st = m.generate(g[f"{name}_prompt"], 16, seq=1, use_graph=use_graph)
        assert list(out) == list(g[f"{name}_greedy"]), use_graph
        assert st["decode_forwards"] == 15


@pytest.mark.parametrize("name", ["tiny", "tiny-q6k"])
def test_tree_batch_golden(models, golden, name):
    """Decode token + chain/alt tree of sequence 0 and a prompt chunk of sequence 1 in one forward (17 tokens: the
    Q6_K model takes the wide-panel arithmetic)."""
    g = golden("models.npz")
    m = models[name]
    m.forward(g[f"{name}_prompt"], 0)
    for step, t in enumerate(g[f"{name}_greedy"]):
        m.forward(np.array([t], np.int32), 24 + step)
    batch = g[f"{name}_tree_batch"].astype(np.int32).view(mk_.BATCH_TOKEN).reshape(-1)
    assert np.array_equal(bits(m.forward_batch(batch)), bits(g[f"{name}_tree_logits"]))
    t1, t2 = m.forward_top2(batch)
    lg = g[f"{name}_tree_logits"]
    for r in range(len(t1)):
        rest = lg[r].copy()
        rest[np.argmax(rest)] = -np.inf
        assert t1[r] == np.argmax(lg[r]) and t2[r] == np.argmax(rest)


def test_against_oracle_multiseq(mk, oracle, model_files):
    """Fresh inputs: 3 sequences, mixed batch, tree through both entry points, move_kv, KV rows byte-identical."""
    rng = np.random.default_rng(21)
    for name in ("tiny", "tiny-tied"):
        dm = mk_.Model(mk, model_files[name], 128, 3)
        om = oracle.model(model_files[name], 128, 3)
        V = dm.cfg["n_vocab"]
        for s in range(3):
            p = rng.integers(0, V, 20 + 3 * s).astype(np.int32)
            assert np.array_equal(bits(dm.forward(p, 0, seq=s)), bits(om.forward(p, 0, seq=s)))
        b = [(5, 0, 20, 1, -1, -1), (7, 1, 23, 1, -1, -1), (9, 1, 24, 1, 24, 1), (11, 1, 24, 1, 25, 1),
             (13, 1, 25, 1, 26, 2)] + [(int(t), 2, 26 + j, int(j == 3), -1, -1) for j, t in
                                       enumerate(rng.integers(0, V, 4))]
        batch = np.array(b, dtype=mk_.BATCH_TOKEN)
        assert np.array_equal(bits(dm.forward_batch(batch)), bits(om.forward_batch(batch)))
        for layer in (0, dm.cfg["n_layer"] - 1):
            for pos in (0, 24, 26):
                for k in (True, False):
                    assert np.array_equal(dm.kv_row(layer, 1, pos, k), om.kv_row(layer, 1, pos, k)), (layer, pos, k)
        dm.move_kv(26, 24, 1)
        om.move_kv(26, 24, 1)
        assert np.array_equal(dm.kv_row(0, 1, 24, True), om.kv_row(0, 1, 24, True))
        nxt = np.array([3, 4], np.int32)
        assert np.array_equal(bits(dm.forward(nxt, 25, seq=1)), bits(om.forward(nxt, 25, seq=1)))
        par = np.array([-1, 0, 0, 1], np.int32)
        tl = rng.integers(0, V, 4).astype(np.int32)
        assert np.array_equal(bits(dm.forward(tl, 27, True, par, 1)), bits(om.forward(tl, 27, True, par, 1)))
        dm.close()
        om.close()


def test_errors_match_reference(mk, oracle, model_files):
    dm = mk_.Model(mk, model_files["tiny"], 64, 2)
    om = oracle.model(model_files["tiny"], 64, 2)
    V = dm.cfg["n_vocab"]
    cases = [
        [(1, 5, 0, 1, -1, -1)],                          # bad slot (sequence)
        [(1, 0, 64, 1, -1, -1)],                         # bad slot (position)
        [(1, 0, 0, 1, -1, -1), (2, 1, 1, 1, 1, 0)],      # parent of another sequence
        [(1, 0, 0, 1, -1, 0)],                           # parent not before the token
        [(V, 0, 0, 1, -1, -1)],                          # token id out of range
    ]
    for c in cases:
        bb = np.array(c, dtype=mk_.BATCH_TOKEN)
        with pytest.raises(mk_.MkError) as ed:
            dm.forward_batch(bb)
        with pytest.raises(RuntimeError) as eo:
            om.forward_batch(bb)
        assert str(ed.value) == str(eo.value), c
        assert ed.value.code == mk_.MK_ERR_INVALID
    with pytest.raises(mk_.MkError, match="context full"):
        dm.forward(np.zeros(10, np.int32), 60)
    with pytest.raises(mk_.MkError, match="batch size out of range"):
        dm.forward_batch(np.zeros(0, dtype=mk_.BATCH_TOKEN))
    # the model still works after errors
    p = np.arange(8, dtype=np.int32)
    assert np.array_equal(bits(dm.forward(p, 0)), bits(om.forward(p, 0)))
    dm.close()
    om.close()


def test_no_wide_q6k(mk, oracle, model_files):
    """MALKIN_NO_WIDE: Q6_K keeps the compact-panel arithmetic above 16 tokens."""
    dm = mk_.Model(mk, model_files["tiny-q6k"], 64, 1, wide=False)
    om = oracle.model(model_files["tiny-q6k"], 64, 1, wide=False)
    p = np.arange(20, dtype=np.int32) * 3
    a, b = dm.forward(p, 0, all_logits=True), om.forward(p, 0, all_logits=True)
    assert np.array_equal(bits(a), bits(b))
    dm.close()
    om.close()


def test_fused_decode_only_for_distinct_sequences(mk, oracle, model_files):
    """A one-token batch (fused QK-norm/RoPE/KV-write/attention) followed by a several-token forward of one sequence
    through the other entry point: the second must not take the fused path (its tokens read each other's new rows)."""
    dm = mk_.Model(mk, model_files["tiny"], 64, 2)
    om = oracle.model(model_files["tiny"], 64, 2)
    b = np.array([(7, 1, 0, 1, -1, -1)], dtype=mk_.BATCH_TOKEN)
    assert np.array_equal(bits(dm.forward_batch(b)), bits(om.forward_batch(b)))
    p = np.array([3, 1, 4], np.int32)
    assert np.array_equal(bits(dm.forward(p, 0, all_logits=True)), bits(om.forward(p, 0, all_logits=True)))
    b2 = np.array([(5, 0, 3, 1, -1, -1), (9, 1, 1, 1, -1, -1)], dtype=mk_.BATCH_TOKEN)  # two sequences: fused
    assert np.array_equal(bits(dm.forward_batch(b2)), bits(om.forward_batch(b2)))
    dm.close()
    om.close()


def test_long_context_against_reference(mk, ref, model_files):
    """A context past one workgroup's LDS (head_dim 128: about 7600 keys): a 16000-token prompt in 256-token forwards,
    a 3-token tree over it and two decode steps, logits bit-identical to the compiled reference's Model."""
    name = "tiny"
    n_ctx = 16400
    dm = mk_.Model(mk, model_files[name], n_ctx, 1)
    rm = ref.model(model_files[name], n_ctx, 1)
    try:
        V = dm.cfg["n_vocab"]
        rng = np.random.default_rng(40)
        p = rng.integers(0, V, 16000).astype(np.int32)
        print("long prompt", len(p), "head_dim", dm.cfg["head_dim"], flush=True)
        for at in range(0, len(p), 256):
            c = p[at:at + 256]
            got, want = dm.forward(c, at), rm.forward(c, at)
            assert np.array_equal(bits(got), bits(want)), at
        par = np.array([-1, 0, 0], np.int32)
        tl = rng.integers(0, V, 3).astype(np.int32)
        assert np.array_equal(bits(dm.forward(tl, 16000, True, par)), bits(rm.forward(tl, 16000, True, par)))
        for step, t in enumerate(rng.integers(0, V, 2)):
            x = np.array([t], np.int32)
            assert np.array_equal(bits(dm.forward(x, 16000 + step)), bits(rm.forward(x, 16000 + step))), step
    finally:
        dm.close()
        rm.close()
