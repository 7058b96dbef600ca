"""Stochastic sampling on the device: mk_penalize / mk_topk against numpy (ties, infinities, row subsets, k up to
1024, vocabularies from 5 to 151936), mk_sampler_distribution / mk_sampler_sample over device rows against the
oracle's Sampler (itself pinned to the compiled reference's in test_sampler.py) with the same seeds and accepted
tokens, and the engine's sampled and penalized requests, with and without a draft model, against the reference
Engine's token loop restated over the oracle's model and sampler (tests/engine_ref.py)."""
import numpy as np
import pytest

import engine_ref
import malkin_amd as mk_

pytestmark = pytest.mark.gpu


def order_key(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def expected_topk(row, k):
    key = order_key(row)
    idx = np.lexsort((np.arange(len(row)), -key.astype(np.int64)))[:k]
    return row[idx], idx


@pytest.mark.parametrize("V", [5, 1024, 151936])
@pytest.mark.parametrize("k", [1, 40, 256, 1024])
def test_topk_vs_numpy(mk, V, k):
    if k > V:
        k = V
    rng = np.random.default_rng(V + k)
    n_rows = 6
    x = (rng.standard_normal((n_rows, V)) * 3).astype(np.float32)
    x[1] = np.round(x[1] * 4) / 4  # many ties: the lower id first
    x[2, ::7] = -np.inf
    x[3, :] = 0.0
    x[3, ::3] = -0.0
    x[4, rng.integers(V)] = np.inf
    rows = np.array([5, 0, 3, 1, 2, 4], np.int32)
    dx, dr = mk.to_device(x), mk.to_device(rows)
    dv, di = mk.alloc(n_rows * k * 4), mk.alloc(n_rows * k * 4)
    print("topk", V, k, flush=True)
    mk_.check(mk_.load().mk_topk(mk.h, dx.ptr, V, dr.ptr, n_rows, V, k, dv.ptr, di.ptr))
    gv = dv.download(np.float32).reshape(n_rows, k)
    gi = di.download(np.int32).reshape(n_rows, k)
    for r in range(n_rows):
        ev, ei = expected_topk(x[rows[r]], k)
        assert np.array_equal(gi[r], ei), (V, k, r)
        assert np.array_equal(gv[r].view(np.uint32), ev.view(np.uint32)), (V, k, r)


def test_penalize_vs_numpy(mk):
    rng = np.random.default_rng(3)
    V, n_rows = 2000, 4
    x = rng.standard_normal((n_rows, V)).astype(np.float32)
    rows = np.array([2, 0, 3, 1], np.int32)
    lists = [[(5, 0.5), (7, 1.25)], [], [(1999, -0.3), (0, 2.0), (5000, 1.0)], [(3, 0.125)]]
    off = np.zeros(n_rows + 1, np.int32)
    ids, amts = [], []
    for r, l in enumerate(lists):
        ids += [i for i, _ in l]
        amts += [a for _, a in l]
        off[r + 1] = len(ids)
    ids, amts = np.array(ids, np.int32), np.array(amts, np.float32)
    dx, dr, do, di, da = mk.to_device(x), mk.to_device(rows), mk.to_device(off), mk.to_device(ids), mk.to_device(amts)
    mk_.check(mk_.load().mk_penalize(mk.h, dx.ptr, V, dr.ptr, n_rows, V, do.ptr, di.ptr, da.ptr))
    got = dx.download(np.float32).reshape(n_rows, V)
    want = x.copy()
    for r, l in enumerate(lists):
        for i, a in l:
            if 0 <= i < V:
                want[rows[r], i] -= np.float32(a)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


GRID = [
    dict(),
    dict(temperature=0.0),
    dict(temperature=0.0, presence=0.7, frequency=0.2),
    dict(top_k=0),
    dict(top_k=1),
    dict(top_k=1024, top_p=0.98, min_p=0.0),
    dict(top_k=2000, top_p=0.8),
    dict(temperature=1.7, top_p=1.0, min_p=0.0),
    dict(temperature=0.3, top_p=0.5, min_p=0.2),
    dict(presence=0.5, frequency=0.3),
]


@pytest.mark.parametrize("V", [1024, 151936])
@pytest.mark.parametrize("params", GRID, ids=[str(g) for g in GRID])
def test_device_distribution_matches_oracle(mk, oracle, V, params):
    """20 steps: each a fresh row, its distribution on the device (penalized in place) and in the oracle, then the
    sampled token accepted by both."""
    rng = np.random.default_rng(V)
    s, a = mk_.Sampler(42, **params), oracle.sampler(42, **params)
    buf = mk.alloc(V * 4)
    print("distribution", V, params, flush=True)
    for step in range(20):
        l = (rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32)
        buf.upload(l)
        d = s.distribution(mk, buf, V)
        la = l.copy()
        e = a.distribution(la)
        assert d == e, (step, d[:4], e[:4])
        assert np.array_equal(buf.download(np.float32).view(np.uint32), la.view(np.uint32)), step
        t1, t2 = s.draw(d), a.draw(e)
        assert t1 == t2, step
        s.accept(t1)
        a.accept(t2)
        buf.upload(l)
        assert s.sample(mk, buf, V) == a.sample(l.copy()), step
    s.close()
    buf.free()


REQUESTS = [
    dict(seed=5),
    dict(seed=6, temperature=1.1, top_k=0, top_p=0.9, presence=0.4, frequency=0.2),
    dict(seed=12, temperature=0.7, top_k=1500, min_p=0.01),
    dict(seed=8, temperature=0.0, frequency=0.6),
    None,  # greedy, no penalties
]


def check_engine(mk, oracle, model_files, draft_name, requests, budget=40, n_ctx=160):
    target = mk_.Model(mk, model_files["tiny"], n_ctx, len(requests))
    draft = mk_.Model(mk, model_files[draft_name], n_ctx, len(requests)) if draft_name else None
    eng = mk_.Engine(target, draft, n_draft=8)
    rng = np.random.default_rng(99)
    prompts = [rng.integers(0, 1024, int(n)).astype(np.int32) for n in rng.integers(3, 40, len(requests))]
    ids = [eng.submit(p, max_tokens=budget, sampling=r) for p, r in zip(prompts, requests)]
    eng.run()
    for rid, p, r in zip(ids, prompts, requests):
        toks, info = eng.result(rid)
        t = oracle.model(model_files["tiny"], n_ctx, 1)
        d = oracle.model(model_files[draft_name], n_ctx, 1) if draft_name else None
        params = dict(r) if r is not None else dict(seed=1, temperature=0.0)
        want, winfo = engine_ref.run_request(oracle, t, d, p, budget, n_ctx, **params)
        t.close()
        if d:
            d.close()
        print("request", rid, draft_name, r, info, winfo, flush=True)
        assert list(toks) == want, (rid, r)
        assert info["drafted"] == winfo["drafted"] and info["accepted"] == winfo["accepted"], (rid, r)
        assert info["finish"] == (1 if winfo["finish"] == "stop" else 0)
    eng.close()
    if draft:
        draft.close()
    target.close()


def test_engine_sampled_requests(mk, oracle, model_files):
    """Sampled, penalized-greedy and plain requests batched together: each stream is the reference loop's for its
    seed."""
    check_engine(mk, oracle, model_files, None, REQUESTS)


@pytest.mark.parametrize("draft_name", ["tiny", "tiny-q4km"])
def test_engine_sampled_speculative(mk, oracle, model_files, draft_name):
    """With a draft: sampled chains verified by Sampler::verify (the draft = the target itself accepts nearly all,
    penalties make the target's distribution differ from the draft's), penalized greedy trees."""
    reqs = [dict(seed=7), dict(seed=11, temperature=0.9, presence=1.5), dict(seed=10, temperature=0.0, frequency=0.6),
            dict(seed=9, temperature=0.6, top_k=300)]
    check_engine(mk, oracle, model_files, draft_name, reqs)


@pytest.mark.parametrize("draft_name", ["tiny", "tiny-q4km"])
def test_engine_sampled_drafts_on_device(mk, oracle, model_files, draft_name):
    """Sampled requests whose draft candidates fit the device's top-k (and whose target rows take no penalties) draw
    their drafts on the device (mk_sample_draw): the step has one host wait however many draft forwards it runs,
    every device draw equals the host's replay of it, and each stream, with its drafted and accepted counts, is the
    reference loop's for its seed."""
    n_ctx, budget = 160, 40
    reqs = [dict(seed=7), dict(seed=9, temperature=0.6, top_k=300), dict(seed=21, temperature=1.3, top_k=1024,
                                                                        top_p=1.0, min_p=0.0)]
    target = mk_.Model(mk, model_files["tiny"], n_ctx, len(reqs))
    draft = mk_.Model(mk, model_files[draft_name], n_ctx, len(reqs))
    eng = mk_.Engine(target, draft, n_draft=8)
    rng = np.random.default_rng(31)
    prompts = [rng.integers(0, 1024, int(n)).astype(np.int32) for n in rng.integers(3, 40, len(reqs))]
    refs = []
    for p, r in zip(prompts, reqs):
        t = oracle.model(model_files["tiny"], n_ctx, 1)
        d = oracle.model(model_files[draft_name], n_ctx, 1)
        refs.append(engine_ref.run_request(oracle, t, d, p, budget, n_ctx, **r))
        t.close()
        d.close()
    # Twice: the first run also grows the engine's buffers (frees wait); the second is measured.
    for run in range(2):
        ids = [eng.submit(p, max_tokens=budget, sampling=r) for p, r in zip(prompts, reqs)]
        mk.sync()
        w0, s0, (dr0, mm0) = mk_.host_waits(), eng.steps, eng.draws
        eng.run()
        waits, steps = mk_.host_waits() - w0, eng.steps - s0
        draws, mismatches = eng.draws[0] - dr0, eng.draws[1] - mm0
        print("draft", draft_name, "run", run, "steps", steps, "host waits", waits, "device draws", draws,
              "mismatches", mismatches, flush=True)
        if run == 1:
            assert steps > 0 and waits == steps
        assert draws > 0 and mismatches == 0
        drafted = 0
        for rid, r, (want, winfo) in zip(ids, reqs, refs):
            toks, info = eng.result(rid)
            print("request", rid, r, info, winfo, flush=True)
            assert list(toks) == want, (rid, r)
            assert info["drafted"] == winfo["drafted"] and info["accepted"] == winfo["accepted"], (rid, r)
            drafted += info["drafted"]
        assert draws == drafted
    eng.close()
    draft.close()
    target.close()


CUT_CASES = [
    (dict(top_k=0), 4.0),                                   # peaked rows: a short kept head
    (dict(top_k=0, temperature=1.3, top_p=0.99, min_p=0.0), 0.5),  # flat rows: a head past the copy's cap
    (dict(top_k=2000, top_p=0.97, min_p=0.0), 1.0),
    (dict(top_k=5000, top_p=1.0, min_p=0.0), 2.0),         # every candidate kept: 5000 > the cap
]


@pytest.mark.parametrize("params,scale", CUT_CASES, ids=[str(c[0]) for c in CUT_CASES])
def test_whole_vocab_cut_on_device(mk, oracle, params, scale):
    """Rows with more than 1024 candidates (top_k <= 0 or above 1024) at V = 151,936 are sorted and cut on the
    device (mk_sample_cut): the distributions and draws equal the oracle's, and what a step downloads is the kept
    head (within the 4096-candidate copy, one wait) instead of the 608 KB row; a head past the copy costs one more
    wait and only its own candidates."""
    V = 151936
    L = mk_.load()
    rng = np.random.default_rng(17)
    s, a = mk_.Sampler(7, **params), oracle.sampler(7, **params)
    buf = mk.alloc(V * 4)
    print("cut", params, scale, flush=True)
    for step in range(6):
        l = (rng.standard_normal(V) * scale).astype(np.float32)
        buf.upload(l)
        w0, b0 = L.mk_host_waits(), L.mk_host_bytes()
        d = s.distribution(mk, buf, V)
        waits, nbytes = L.mk_host_waits() - w0, L.mk_host_bytes() - b0
        e = a.distribution(l.copy())
        assert d == e, (step, len(d), len(e), d[:3], e[:3])
        kept = len(d)
        print("step", step, "kept", kept, "waits", waits, "bytes", nbytes, flush=True)
        head = min(kept + 1, params["top_k"] if params["top_k"] > 0 else V)
        if step > 0:  # the first call also allocates the selector's buffers
            assert waits == (1 if head <= 4096 else 2), waits
        assert nbytes <= 4096 * 8 + 64 + max(0, head - 4096) * 8, nbytes
        if head <= 4096:
            assert nbytes < V * 4 // 16, nbytes
        t1, t2 = s.draw(d), a.draw(e)
        assert t1 == t2, step
        s.accept(t1)
        a.accept(t2)
    s.close()
    buf.free()


DRAW_ROWS = [  # (top_k, temperature, top_p, min_p): per generator
    (40, 0.8, 0.95, 0.05),   # the defaults
    (1, 0.8, 0.95, 0.05),    # one candidate: no draw, the generator untouched
    (1024, 1.5, 1.0, 0.0),   # every candidate kept
    (12, 0.05, 0.9, 0.1),    # peaked: mostly one kept, some draws
    (300, 1.1, 0.5, 0.0),    # nucleus cut inside the candidates
]


def mt_words(g):
    """The oracle generator's state in mk_sample_draw's layout: 312 words, then the index as a word."""
    raw = np.frombuffer(g.state.raw, np.uint64)
    return np.concatenate([raw[:312], np.array([int(np.frombuffer(g.state.raw[312 * 8:312 * 8 + 4], np.int32)[0])],
                                               np.uint64)])


def test_sample_draw_matches_oracle(mk, oracle):
    """mk_sample_draw (the draft's draws on the device) against the oracle's Sampler::distribution + Sampler::draw:
    rows of 1024 candidates with one generator each, 700 calls in a row (every generator that draws regenerates its
    state twice), the ids of every call and the final generator states (words and index) bit-equal."""
    L = mk_.load()
    rng = np.random.default_rng(23)
    G, K, R = len(DRAW_ROWS), 1024, 700
    seeds = [3, 1 << 40, 12345, 0xDEADBEEF, 77]
    gens = [oracle.mt64(s) for s in seeds]
    states = np.stack([mt_words(g) for g in gens])
    dstates = mk.to_device(states)
    params = np.zeros((R, G, 6), np.int32)
    pv = params.view(np.float32)
    vals = np.zeros((R, G, K), np.float32)
    ids = np.zeros((R, G, K), np.int32)
    want = np.zeros((R, G), np.int32)
    for r in range(R):
        for g, (k, t, tp, mp) in enumerate(DRAW_ROWS):
            l = (rng.standard_normal(K) * rng.uniform(0.5, 3)).astype(np.float32)
            e = oracle.sampler(1, top_k=k, temperature=t, top_p=tp, min_p=mp).distribution(l.copy())
            want[r, g] = oracle_draw(oracle, gens[g], e)
            order = np.lexsort((np.arange(K), -l.astype(np.float64)))
            vals[r, g], ids[r, g] = l[order], order
            params[r, g, 0] = k
            pv[r, g, 1:4] = (t, mp, tp)
            params[r, g, 4] = g
            params[r, g, 5] = r * G + g
    dv, di, dp = mk.to_device(vals), mk.to_device(ids), mk.to_device(params)
    dout = mk.alloc(R * G * 4)
    print("sample_draw", G, K, R, flush=True)
    for r in range(R):
        off = r * G
        mk_.check(L.mk_sample_draw(mk.h, dv.offset(off * K * 4), di.offset(off * K * 4), K, G, dp.offset(off * 24),
                                   dstates.ptr, G, dout.ptr, R * G))
    got = dout.download(np.int32).reshape(R, G)
    for g in range(G):
        bad = np.nonzero(got[:, g] != want[:, g])[0]
        assert bad.size == 0, (DRAW_ROWS[g], int(bad[0]), got[bad[0], g], want[bad[0], g])
    assert np.array_equal(dstates.download(np.uint64).reshape(G, 313), np.stack([mt_words(g) for g in gens]))
    assert mt_words(gens[1])[312] == 312 and np.array_equal(mt_words(gens[1]), states[1])  # k = 1 drew nothing
    for b in (dv, di, dp, dout, dstates):
        b.free()


def oracle_draw(oracle, g, d):
    pp = np.array([p for p, _ in d], np.float32)
    pi = np.array([i for _, i in d], np.int32)
    return int(oracle.lib.or_draw(g.state, pp.ctypes.data, pi.ctypes.data, len(pp)))


def test_sample_draw_edges(mk, oracle):
    """mk_sample_draw's boundaries: a row whose generator or destination index is out of range is skipped (its
    output and every generator untouched), k is clamped to 1..stride (k <= 0 and k > stride draw as 1 and stride
    candidates), stride 1 always picks the only candidate without drawing, and a stride above 1024 is refused with
    a status before anything is queued."""
    L = mk_.load()
    rng = np.random.default_rng(29)
    K, G = 16, 2
    gens = [oracle.mt64(101), oracle.mt64(202)]
    states = np.stack([mt_words(g) for g in gens])
    dstates = mk.to_device(states)
    l = np.sort(rng.standard_normal((4, K)).astype(np.float32), axis=1)[:, ::-1].copy()
    ids = np.tile(np.arange(K, dtype=np.int32) * 3, (4, 1))
    dv, di = mk.to_device(l), mk.to_device(ids)
    # rows: 0 bad state, 1 bad dst, 2 k = 0 (one candidate), 3 k = 99 (all 16) from generator 1
    params = np.zeros((4, 6), np.int32)
    pv = params.view(np.float32)
    pv[:, 1:4] = (1.0, 0.0, 1.0)  # temperature 1, min_p 0, top_p 1
    params[:, 0] = (K, K, 0, 99)
    params[:, 4] = (G, 0, 0, 1)
    params[:, 5] = (0, 4, 2, 3)
    out0 = np.full(4, -7, np.int32)
    dp, dout = mk.to_device(params), mk.to_device(out0)
    mk_.check(L.mk_sample_draw(mk.h, dv.ptr, di.ptr, K, 4, dp.ptr, dstates.ptr, G, dout.ptr, 4))
    got = dout.download(np.int32)
    assert got[0] == -7 and got[1] == -7, got  # skipped rows wrote nothing
    assert got[2] == ids[2, 0]                  # one candidate: no draw
    e = oracle.sampler(1, top_k=K, temperature=1.0, top_p=1.0, min_p=0.0).distribution(
        np.ascontiguousarray(l[3][np.argsort(ids[3] // 3)]))
    e = [(p, int(ids[3][i])) for p, i in e]
    assert got[3] == oracle_draw(oracle, gens[1], e)
    after = dstates.download(np.uint64).reshape(G, 313)
    assert np.array_equal(after[0], states[0])  # generator 0 served only skipped / one-candidate rows
    assert np.array_equal(after[1], mt_words(gens[1]))
    # stride 1: the only candidate, generator untouched
    params1 = np.array([[5, 0, 0, 0, 0, 0]], np.int32)
    params1.view(np.float32)[0, 1:4] = (1.0, 0.0, 1.0)
    dp1 = mk.to_device(params1)
    mk_.check(L.mk_sample_draw(mk.h, dv.ptr, di.ptr, 1, 1, dp1.ptr, dstates.ptr, G, dout.ptr, 4))
    assert dout.download(np.int32)[0] == ids[0, 0]
    assert np.array_equal(dstates.download(np.uint64).reshape(G, 313)[0], states[0])
    # a stride above mk_topk's 1024 is refused
    rc = L.mk_sample_draw(mk.h, dv.ptr, di.ptr, 1025, 1, dp1.ptr, dstates.ptr, G, dout.ptr, 4)
    assert rc == mk_.MK_ERR_INVALID and "1024" in L.mk_last_error().decode()
    for b in (dv, di, dp, dp1, dout, dstates):
        b.free()
