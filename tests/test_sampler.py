"""Stochastic sampling on the CPU: the oracle's restatement of the reference's Sampler (oracle.c, sampler.cpp:22-141)
pinned by the C++ standard's known answer for std::mt19937_64, by closed forms (softmax, min-p floor, nucleus
boundary), by the compiled reference's own Sampler (oracle/_ref) on the same logits and seeds, and by the
reference's own exactness experiment for speculative verification (test_sampler.cpp: total variation < 0.005);
then the product's host half (mk_sampler_draw / mk_sampler_verify, no device needed) against the oracle, and the
single-request engine restatement (tests/engine_ref.py) with the oracle's model and sampler against the same
restatement over the compiled reference's."""
import numpy as np
import pytest

import engine_ref

GRID = [
    dict(),
    dict(temperature=0.0),
    dict(temperature=0.0, presence=0.7, frequency=0.2),
    dict(top_k=0),
    dict(top_k=1),
    dict(top_k=2000, top_p=0.8),
    dict(temperature=1.7, top_p=1.0, min_p=0.0),
    dict(temperature=0.3, top_p=0.5, min_p=0.2),
    dict(presence=0.5, frequency=0.3),
    dict(presence=-0.4, frequency=0.1, top_k=0, top_p=0.99),
]


def rows(seed, n, V):
    rng = np.random.default_rng(seed)
    return [(rng.standard_normal(V) * rng.uniform(0.5, 4)).astype(np.float32) for _ in range(n)]


def test_mt19937_64_known_answer(oracle):
    """[rand.predef]: the 10000th output of a default-seeded (5489) std::mt19937_64 is 9981545732273789042."""
    g = oracle.mt64(5489)
    for _ in range(9999):
        g.next()
    assert g.next() == 9981545732273789042
    # uniform(): one output scaled by 2^-64 (closed form on a fresh generator with the same seed)
    a, b = oracle.mt64(12345), oracle.mt64(12345)
    for _ in range(1000):
        x = a.next()
        u = b.uniform()
        assert u == min(float(x) / 2.0 ** 64, np.nextafter(1.0, 0.0)) and 0.0 <= u < 1.0


def test_distribution_closed_forms(oracle):
    V = 3000
    for l in rows(1, 5, V):
        # no cut: softmax of l / T over the whole vocabulary, highest first
        T = 1.3
        d = oracle.sampler(1, top_k=0, top_p=1.0, min_p=0.0, temperature=T).distribution(l.copy())
        assert len(d) == V
        e = np.exp((l.astype(np.float64) - l.max()) / T)
        p = e / e.sum()
        ids = np.array([i for _, i in d])
        assert np.array_equal(ids, np.lexsort((np.arange(V), -l)))
        assert np.allclose([q for q, _ in d], p[ids], rtol=1e-5, atol=1e-9)
        # top-k 1 and greedy: the first maximum
        assert oracle.sampler(1, top_k=1).distribution(l.copy()) == [(1.0, int(np.argmax(l)))]
        assert oracle.sampler(1, temperature=0.0).distribution(l.copy()) == [(1.0, int(np.argmax(l)))]
        # min-p: every kept weight is at least min_p times the first; the first dropped one (if min-p dropped it)
        # is below
        mp = 0.3
        d = oracle.sampler(1, top_k=0, top_p=1.0, min_p=mp, temperature=1.0).distribution(l.copy())
        w = np.sort(np.exp(l.astype(np.float64) - l.max()))[::-1]
        assert len(d) == int((w >= mp * w[0] * (1 - 1e-6)).sum()) or abs(w[len(d)] - mp) < 1e-6
        # nucleus: the kept head's weight reaches top_p of the total, without its last entry it does not
        tp = 0.6
        d = oracle.sampler(1, top_k=0, top_p=tp, min_p=0.0, temperature=1.0).distribution(l.copy())
        n = len(d)
        assert w[:n].sum() >= tp * w.sum() * (1 - 1e-6) and w[:n - 1].sum() < tp * w.sum() * (1 + 1e-6)
        assert abs(sum(q for q, _ in d) - 1.0) < 1e-5


def test_penalties_closed_form(oracle):
    l = rows(2, 1, 100)[0]
    s = oracle.sampler(3, temperature=0.0, presence=0.5, frequency=0.25)
    for t in (7, 7, 9, 7):
        s.accept(t)
    x = l.copy()
    s.distribution(x)
    want = l.copy()
    want[7] -= np.float32(0.5 + 0.25 * 3)
    want[9] -= np.float32(0.5 + 0.25 * 1)
    assert np.array_equal(x, want)


@pytest.mark.parametrize("params", GRID, ids=[str(g) for g in GRID])
def test_oracle_matches_reference_sampler(oracle, ref, params):
    """Same logits, same seed: the oracle's distributions, draws and (penalized) logits equal the compiled
    reference's Sampler for 40 steps, each step accepting the drawn token."""
    a, b = oracle.sampler(42, **params), ref.sampler(42, **params)
    for step, l in enumerate(rows(7, 40, 1500)):
        la, lb = l.copy(), l.copy()
        da, db = a.distribution(la), b.distribution(lb)
        assert da == db, step
        assert np.array_equal(la.view(np.uint32), lb.view(np.uint32)), step
        ta, tb = a.draw(da), b.draw(db)
        assert ta == tb, step
        a.accept(ta)
        b.accept(tb)


def random_pq(rng, V, miss=None):
    p = rng.random(V).astype(np.float32)
    q = rng.random(V).astype(np.float32)
    if miss is not None:
        q[miss] = 0.0
    p /= p.sum()
    q /= q.sum()
    P = [(float(x), i) for i, x in enumerate(p)]
    Q = [(float(x), i) for i, x in enumerate(q) if x > 0]
    return P, Q


def test_oracle_verify_matches_reference(oracle, ref):
    rng = np.random.default_rng(5)
    a, b = oracle.sampler(9), ref.sampler(9)
    for it in range(3000):
        V = int(rng.integers(2, 12))
        P, Q = random_pq(rng, V, miss=int(rng.integers(V)))
        d = int(rng.integers(V))
        assert a.verify(P, Q, d) == b.verify(P, Q, d), it
        assert a.draw(P) == b.draw(P), it


def test_verify_is_exact(oracle):
    """test_sampler.cpp:20-51: drafts d ~ q verified against p come out distributed as p (total variation below
    0.005 over 400000 draws, five trials, q missing one token p has)."""
    rng = np.random.default_rng(7)
    V, N = 8, 400000
    for trial in range(5):
        P, Q = random_pq(rng, V, miss=trial)
        hist, acc = oracle.verify_experiment(P, Q, 11 + trial, 99 + trial, N, V)
        tv = 0.5 * sum(abs(hist[i] / N - p) for p, i in P)
        print("trial", trial, "tv", tv, "accepted", acc / N)
        assert tv < 0.005
        assert 0 < acc < N


def test_product_host_sampler_matches_oracle(oracle):
    """mk_sampler_draw / mk_sampler_verify (the library's host half) draw the oracle's stream for the same seed."""
    import malkin_amd as mk_
    rng = np.random.default_rng(8)
    s, a = mk_.Sampler(77), oracle.sampler(77)
    for it in range(3000):
        V = int(rng.integers(1, 12))
        P, Q = random_pq(rng, V, miss=int(rng.integers(V)) if V > 1 else None)
        d = int(rng.integers(V))
        assert s.draw(P) == a.draw(P), it
        assert s.verify(P, Q, d) == a.verify(P, Q, d), it
    s.close()


CASES = [
    ("tiny", None, dict(seed=5)),
    ("tiny", None, dict(seed=6, temperature=1.1, top_k=0, top_p=0.9, presence=0.4, frequency=0.2)),
    ("tiny", "tiny-q4km", dict(seed=7)),
    ("tiny", "tiny-q4km", dict(seed=8, temperature=0.0, frequency=0.6)),
    ("tiny", "tiny", dict(seed=9, temperature=0.6, top_k=300)),
    ("tiny", "tiny", dict(seed=10, temperature=0.0, frequency=0.6)),
    ("tiny", "tiny", dict(seed=11, temperature=0.9, presence=1.5)),
]


@pytest.mark.parametrize("tname,dname,params", CASES)
def test_engine_restatement_oracle_vs_reference(oracle, ref, model_files, tname, dname, params):
    """The engine restatement gives the same stream and counters over the oracle's model and sampler as over the
    compiled reference's Model and Sampler."""
    rng = np.random.default_rng(params["seed"])
    prompt = rng.integers(0, 1024, 19).astype(np.int32)
    res = []
    for cpu in (oracle, ref):
        t = cpu.model(model_files[tname], 160, 1)
        d = cpu.model(model_files[dname], 160, 1) if dname else None
        res.append(engine_ref.run_request(cpu, t, d, prompt, 40, 160, **params))
        t.close()
        if d:
            d.close()
    print(res[0])
    assert res[0] == res[1]
    assert len(res[0][0]) > 0
