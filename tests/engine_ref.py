"""One request through the reference Engine's token loop, restated over a CPU model and sampler (the oracle's, or
the compiled reference's from oracle/_ref): the checker for the device engine's streams. TEST INFRASTRUCTURE.

Follows /root/reference/src/engine.cpp for a single busy slot (sequence 0):
  * prompt: one forward, the first token sampled from the last row (engine.cpp:407-418);
  * draft depth kk = max(0, min(k, left, free, cap)), free and cap halved for greedy requests, with
    free = n_ctx - cached - 2 and cap = 256 / 1 - 1 (engine.cpp:336-356);
  * drafting (engine.cpp:283-334): catch-up of the draft's cache to cache + next with prefix reuse, then kk picks:
    greedy = top-1 chain with the runner-up as alternative, sampled = draws of the draft sampler (seed + 1, no
    penalties) from its distribution;
  * the target batch (engine.cpp:358-372): greedy [next, chain_0, alt_0, ...] as a tree, sampled [next, d_0, ...];
  * acceptance (engine.cpp:423-501): the greedy walk over the penalized argmax with KV moves, or Sampler::verify per
    draft; adaptive k; emit (engine.cpp:57-70) counts every emitted token into the sampler's penalties.
"""
import numpy as np

from oracle import bind

K_MAX_BATCH = 256


def common_prefix(a, b):
    n = 0
    while n < len(a) and n < len(b) and a[n] == b[n]:
        n += 1
    return n


def top2(l):
    """engine.cpp:309-318: first maximum and the strict runner-up scan."""
    a, b = 0, 1
    if l[b] > l[a]:
        a, b = b, a
    for v in range(2, len(l)):
        if l[v] > l[a]:
            b, a = a, v
        elif l[v] > l[b]:
            b = v
    return a, b


def chunked(m, toks, pos):
    """The last row of tokens fed from position pos in forwards of at most K_MAX_BATCH tokens, as the reference
    engine feeds a prompt (one chunk per step, engine.cpp:359-381) and a draft's catch-up (passes flushed when full,
    engine.cpp:283-298): where the arithmetic depends on a forward's size (Q6_K's wide panels past 16 tokens), the
    chunking decides the row."""
    toks = np.asarray(toks, np.int32)
    last = None
    for i in range(0, len(toks), K_MAX_BATCH):
        last = m.forward(toks[i:i + K_MAX_BATCH], pos + i)[-1].copy()
    return last


def run_request(cpu, target, draft, prompt, max_tokens, n_ctx, seed, eog=(), n_draft=8, **params):
    """cpu: bind.Oracle() or bind.Ref(); target / draft: its models (draft may be None) with a fresh sequence 0.
    Returns (tokens, info) with the engine's counters."""
    p = dict(bind.SAMPLING_DEFAULTS, **params)
    greedy = p["temperature"] <= 0
    S = cpu.sampler(seed, True, **params)
    DS = cpu.sampler(seed + 1 if seed else 0, False, **params)
    budget = max_tokens if max_tokens > 0 else n_ctx
    out, info = [], dict(drafted=0, accepted=0, finish="length")
    cache, dcache = [int(t) for t in prompt], []
    k = min(4, n_draft)

    def emit(t):
        if t in eog:
            info["finish"] = "stop"
            return False
        S.accept(t)
        out.append(t)
        if len(out) >= budget:
            return False
        return len(cache) + 1 < n_ctx

    last = chunked(target, prompt, 0)
    nxt = S.sample(last)
    alive = emit(nxt)
    while alive:
        P = len(cache)
        kk = 0
        if draft is not None:
            left, free, cap = budget - len(out), n_ctx - P - 2, K_MAX_BATCH // 1 - 1
            kk = max(0, min(k, left, free // 2 if greedy else free, cap // 2 if greedy else cap))
        chain, alt, qd = [], [], []
        if kk > 0:
            L = P + 1
            common = common_prefix(dcache, cache)
            if common == len(cache) and common < len(dcache) and dcache[common] == nxt:
                common += 1
            common = min(common, L - 1)
            dcache = dcache[:common]
            toks = [cache[q] if q < P else nxt for q in range(common, L)]
            dl = chunked(draft, toks, common)
            dcache += toks
            for i in range(kk):
                if greedy:
                    a, b = top2(dl)
                    alt.append(b)
                else:
                    q = DS.distribution(dl)
                    qd.append(q)
                    a = DS.draw(q)
                chain.append(a)
                if i + 1 < kk:
                    dl = draft.forward(np.asarray([a], np.int32), len(dcache))[-1].copy()
                    dcache.append(a)
        batch = [(nxt, 0, P, 1, -1, -1)]
        for i in range(kk):
            if greedy:
                par = 0 if i == 0 else 2 * i - 1
                batch.append((chain[i], 0, P + 1 + i, 1, P + 1 + 2 * i, par))
                batch.append((alt[i], 0, P + 1 + i, 1, P + 2 + 2 * i, par))
            else:
                batch.append((chain[i], 0, P + 1 + i, 1, -1, -1))
        bt = np.zeros(len(batch), dtype=bind.BATCH_TOKEN)
        for j, t in enumerate(batch):
            bt[j] = t
        rows = target.forward_batch(bt)
        cache.append(nxt)
        info["drafted"] += kk
        go = True
        if kk == 0:
            nxt = S.sample(rows[0].copy())
        elif greedy:
            cur, done, bonus = 0, 0, False
            for i in range(kk):
                a = S.distribution(rows[cur].copy())[0][1]
                slot = 1 + 2 * i if a == chain[i] else 2 + 2 * i if a == alt[i] else -1
                if slot < 0:
                    nxt, bonus = a, True
                    break
                target.move_kv(P + slot, len(cache), 0)
                cache.append(a)
                info["accepted"] += 1
                cur = slot
                go = emit(a)
                if not go:
                    break
                done = i + 1
                if slot == 2 + 2 * i:
                    break
            if go and not bonus:
                nxt = S.distribution(rows[cur].copy())[0][1]
            if done == kk and kk == k and cur == 2 * kk - 1:
                k = min(k + 1, n_draft)
            elif 2 * done < kk:
                k = max(1, k - 1)
        else:
            i = 0
            while i < kk:
                t, ok = S.verify(S.distribution(rows[i].copy()), qd[i], chain[i])
                if not ok:
                    nxt = t
                    break
                info["accepted"] += 1
                cache.append(t)
                go = emit(t)
                if not go:
                    break
                i += 1
            if go and i == kk:
                nxt = S.sample(rows[kk].copy())
            if i == kk and kk == k:
                k = min(k + 1, n_draft)
            elif 2 * i < kk:
                k = max(1, k - 1)
        if go:
            go = emit(nxt)
        alive = go
    return out, info
