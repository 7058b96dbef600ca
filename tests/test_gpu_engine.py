"""The device token loop (include/malkin_engine.h) against plain greedy decoding, the invariants the reference holds
for its Engine: continuous batching of several sequences produces each sequence's own greedy stream
(tools/check_parallel.sh: batched greedy == sequential greedy), and greedy speculative decoding with a draft's
chain/runner-up tree produces exactly the target's greedy stream (README.md:36). Plain greedy streams come from
Model.generate, which the model tests pin to the CPU oracle."""
import numpy as np
import pytest

import malkin_amd as mk_

pytestmark = pytest.mark.gpu


def plain(mk, path, prompt, n):
    m = mk_.Model(mk, path, 160, 1)
    toks, _ = m.generate(np.asarray(prompt, np.int32), n, use_graph=False)
    m.close()
    return list(toks)


def prompts(rng, V, lens):
    return [rng.integers(0, V, n).astype(np.int32) for n in lens]


def test_engine_continuous_batching(mk, model_files):
    path = model_files["tiny"]
    target = mk_.Model(mk, path, 160, 4)
    V = target.cfg["n_vocab"]
    rng = np.random.default_rng(11)
    ps = prompts(rng, V, [5, 40, 17, 1, 29, 9])
    budgets = [12, 8, 20, 10, 6, 15]
    eng = mk_.Engine(target)
    ids = [eng.submit(p, max_tokens=b) for p, b in zip(ps, budgets)]
    eng.run()
    for rid, p, b in zip(ids, ps, budgets):
        toks, info = eng.result(rid)
        print("request", rid, len(p), b, info, flush=True)
        assert info["done"] == 1 and info["finish"] == 0
        assert info["prompt_tokens"] == len(p) and info["completion_tokens"] == b
        assert list(toks) == plain(mk, path, p, b), rid
    # the last admitted prompt again (its slot was not reused since): its KV prefix is reused (all but the last
    # prompt token), same stream
    rid = eng.submit(ps[5], max_tokens=8)
    eng.run()
    toks, info = eng.result(rid)
    assert info["cached_tokens"] == len(ps[5]) - 1
    assert list(toks) == plain(mk, path, ps[5], 8)
    eng.close()
    target.close()


@pytest.mark.parametrize("draft_name", ["tiny", "tiny-q4km"])
def test_engine_speculative_greedy(mk, model_files, draft_name):
    """Draft = the target itself (every draft accepted: KV moves along the chain) or a differently quantized model
    (rejections, runner-up leaves): the accepted streams equal plain greedy either way."""
    path = model_files["tiny"]
    target = mk_.Model(mk, path, 160, 3)
    draft = mk_.Model(mk, model_files[draft_name], 160, 3)
    V = target.cfg["n_vocab"]
    rng = np.random.default_rng(12)
    ps = prompts(rng, V, [7, 33, 20])
    budgets = [30, 25, 40]
    eng = mk_.Engine(target, draft, n_draft=8)
    ids = [eng.submit(p, max_tokens=b) for p, b in zip(ps, budgets)]
    eng.run()
    drafted = accepted = 0
    for rid, p, b in zip(ids, ps, budgets):
        toks, info = eng.result(rid)
        print("request", rid, draft_name, info, flush=True)
        assert info["completion_tokens"] == b
        assert list(toks) == plain(mk, path, p, b), (draft_name, rid)
        drafted += info["drafted"]
        accepted += info["accepted"]
    assert drafted > 0
    if draft_name == "tiny":
        assert accepted > 0.8 * drafted  # the draft is the target: only budget edges cut chains short
    eng.close()
    draft.close()
    target.close()


def test_engine_eog_and_errors(mk, model_files):
    path = model_files["tiny"]
    target = mk_.Model(mk, path, 64, 2)
    p = np.array([3, 14, 15, 92, 65], np.int32)
    ref = plain(mk, path, p, 6)
    eng = mk_.Engine(target)
    rid = eng.submit(p, max_tokens=20, eog=[ref[2]])
    eng.run()
    toks, info = eng.result(rid)
    stop_at = ref.index(ref[2])
    assert list(toks) == ref[:stop_at] and info["finish"] == 1
    with pytest.raises(mk_.MkError, match="empty prompt"):
        eng.submit(np.zeros(0, np.int32))
    with pytest.raises(mk_.MkError, match="prompt has 64 tokens, context is 64"):
        eng.submit(np.zeros(64, np.int32))
    # the context end finishes a request ("length") one token before the last KV row
    rid = eng.submit(np.arange(60, dtype=np.int32) % 7, max_tokens=0)
    eng.run()
    toks, info = eng.result(rid)
    assert info["finish"] == 0 and info["completion_tokens"] == 64 - 60
    eng.close()
    target.close()


@pytest.mark.parametrize("draft_name", [None, "tiny", "tiny-q4km"])
def test_engine_one_host_wait_per_step(mk, model_files, draft_name):
    """The step's draft rounds, tree layout, acceptance moves and next prompt chunks run without the host waiting in
    between: the library's host waits (stream / event synchronizations) equal the engine's steps."""
    path = model_files["tiny"]
    target = mk_.Model(mk, path, 160, 3)
    draft = mk_.Model(mk, model_files[draft_name], 160, 3) if draft_name else None
    V = target.cfg["n_vocab"]
    ps = prompts(np.random.default_rng(13), V, [9, 50, 21])
    eng = mk_.Engine(target, draft, n_draft=8)
    ids = [eng.submit(p, max_tokens=24) for p in ps]
    mk.sync()
    w0, s0 = mk_.host_waits(), eng.steps
    eng.run()
    waits, steps = mk_.host_waits() - w0, eng.steps - s0
    print("draft", draft_name, "steps", steps, "host waits", waits, flush=True)
    assert steps > 0 and waits == steps
    for rid, p in zip(ids, ps):
        toks, _ = eng.result(rid)
        assert list(toks) == plain(mk, path, p, 24), (draft_name, rid)
    eng.close()
    if draft:
        draft.close()
    target.close()
