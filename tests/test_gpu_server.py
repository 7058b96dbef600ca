"""The HTTP API over the device engine (include/malkin_server.h): concurrent completions, greedy and sampled, plain and
streamed, give the token streams of the reference's engine loop (tests/engine_ref.py over the oracle's model and
sampler), with the reference's usage / timings fields; end-of-generation ids stop a request; a client that goes
away mid-stream cancels its request and the server keeps serving; the engine is usable again after the server
stops."""
import http.client
import json
import socket
import threading

import numpy as np
import pytest

import engine_ref
import malkin_amd as mk_

pytestmark = pytest.mark.gpu

N_CTX = 160


def post(port, body, stream=False):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=120)
    c.request("POST", "/v1/completions", body=json.dumps(body).encode(), headers={"Content-Type": "application/json"})
    r = c.getresponse()
    if not stream:
        out = r.status, json.loads(r.read().decode())
        c.close()
        return out
    events = []
    for raw in r.read().decode().split("\n\n"):
        if raw.startswith("data: "):
            events.append(raw[6:])
    c.close()
    return r.status, events


def expected(oracle, model_files, prompt, max_tokens, sampling, eog=()):
    t = oracle.model(model_files["tiny"], N_CTX, 1)
    try:
        params = dict(sampling) if sampling else dict(temperature=0.0)
        params.setdefault("seed", 1)  # greedy requests draw nothing
        return engine_ref.run_request(oracle, t, None, prompt, max_tokens, N_CTX, eog=tuple(eog), **params)
    finally:
        t.close()


def test_server_completions(mk, oracle, model_files):
    target = mk_.Model(mk, model_files["tiny"], N_CTX, 3)
    eng = mk_.Engine(target)
    srv = mk_.Server(eng, model_id="tiny")
    rng = np.random.default_rng(21)
    cases = [
        (dict(temperature=0.0), 20, False),
        (dict(seed=31, temperature=0.9, top_k=50), 24, False),
        (dict(seed=32, temperature=0.7, presence=0.3), 18, True),
        (dict(seed=33), 22, True),
        (dict(temperature=0.0, frequency=0.5), 16, True),
    ]
    prompts = [rng.integers(0, 1024, int(n)).astype(np.int32) for n in rng.integers(4, 30, len(cases))]
    results = [None] * len(cases)

    def fields(s):
        out = {}
        for k, v in s.items():
            out[{"presence": "presence_penalty", "frequency": "frequency_penalty"}.get(k, k)] = v
        return out

    def worker(i):
        s, n, stream = cases[i]
        body = dict(prompt=[int(x) for x in prompts[i]], max_tokens=n, stream=stream, **fields(s))
        results[i] = post(srv.port, body, stream)

    try:
        threads = [threading.Thread(target=worker, args=(i,)) for i in range(len(cases))]
        for t in threads:
            t.start()
        for t in threads:
            t.join(timeout=300)
        for i, (s, n, stream) in enumerate(cases):
            print("case", i, s, n, stream, flush=True)
            want, winfo = expected(oracle, model_files, prompts[i], n, s)
            st, r = results[i]
            assert st == 200, r
            if not stream:
                ch = r["choices"][0]
                assert ch["tokens"] == want and ch["finish_reason"] == winfo["finish"]
                assert r["object"] == "text_completion" and r["model"] == "tiny"
                assert r["usage"]["completion_tokens"] == len(want) and r["usage"]["prompt_tokens"] == len(prompts[i])
                assert r["timings"]["predicted_n"] == len(want)
            else:
                assert r[-1] == "[DONE]"
                evs = [json.loads(e) for e in r[:-1]]
                toks = [t for e in evs for t in e["choices"][0]["tokens"]]
                assert toks == want
                assert all(e["choices"][0]["finish_reason"] is None for e in evs[:-1])
                assert evs[-1]["choices"][0]["finish_reason"] == winfo["finish"]
                assert evs[-1]["usage"]["completion_tokens"] == len(want)
        # end-of-generation ids: the stream stops before the first one (not emitted), finish "stop"
        s, n = dict(seed=34, temperature=1.0, top_k=0), 30
        want, _ = expected(oracle, model_files, prompts[0], n, s)
        stop_id = want[5]
        st, r = post(srv.port, dict(prompt=[int(x) for x in prompts[0]], max_tokens=n, stop_token_ids=[stop_id],
                                    seed=34, temperature=1.0, top_k=0))
        want_eog, winfo = expected(oracle, model_files, prompts[0], n, s, eog=[stop_id])
        assert st == 200 and r["choices"][0]["tokens"] == want_eog and r["choices"][0]["finish_reason"] == "stop"
        assert stop_id not in want_eog
        # refusals: the engine's texts as 400s
        st, r = post(srv.port, dict(prompt=[]))
        assert st == 400 and "empty prompt" in r["error"]["message"]
        st, r = post(srv.port, dict(prompt=[1] * N_CTX))
        assert st == 400 and "context" in r["error"]["message"]
        st, r = post(srv.port, dict(prompt=[5000]))
        assert st == 400 and "vocabulary" in r["error"]["message"]
        # a streaming client that disconnects after the first event: cancelled, the server carries on
        with socket.create_connection(("127.0.0.1", srv.port), timeout=60) as sk:
            body = json.dumps(dict(prompt=[1, 2, 3], max_tokens=120, stream=True, temperature=0.0)).encode()
            sk.sendall(b"POST /v1/completions HTTP/1.1\r\nContent-Length: " + str(len(body)).encode() + b"\r\n\r\n" +
                       body)
            got = b""
            while b"data: " not in got:
                part = sk.recv(4096)
                assert part, got
                got += part
        st, r = post(srv.port, dict(prompt=[int(x) for x in prompts[1]], max_tokens=8, temperature=0.0))
        want, _ = expected(oracle, model_files, prompts[1], 8, None)
        assert st == 200 and r["choices"][0]["tokens"] == want
    finally:
        srv.close()
    # the engine is the caller's again
    rid = eng.submit(prompts[2], max_tokens=6)
    eng.run()
    toks, info = eng.result(rid)
    want, _ = expected(oracle, model_files, prompts[2], 6, None)
    assert list(toks) == want
    eng.close()
    target.close()


def test_model_eog_stops_requests(mk, oracle, model_files, tmp_path, synth_lib):
    """The model's own end-of-generation id (tokenizer.ggml.eos_token_id) ends a request that lists no stop ids,
    finish "stop", as the reference's engine stops at Tokenizer::is_eog for every request (engine.cpp:60); the server
    frees each finished result; out-of-range integer fields are refused and negative seeds wrap as get<uint64_t>()
    makes them."""
    import make_golden
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, 1024, 12).astype(np.int32)
    want, _ = expected(oracle, model_files, prompt, 24, None)
    # the first token of the greedy stream, from the fourth on, that has not appeared before it
    i = next(i for i in range(3, len(want)) if want[i] not in want[:i])
    eos = want[i]
    c = make_golden.MODEL_CFGS["tiny"]
    path = str(tmp_path / "tiny-eos.gguf")
    synth_lib.write_gguf(path, synth_lib.make_config(c["preset"], c["wtype"], seed=c["seed"], eos_id=eos), threads=4)
    target = mk_.Model(mk, path, N_CTX, 2)
    assert target.eog == [eos]
    eng = mk_.Engine(target)
    srv = mk_.Server(eng, model_id="tiny-eos")
    try:
        st, r = post(srv.port, dict(prompt=[int(x) for x in prompt], max_tokens=24, temperature=0.0))
        print("eos", eos, "at", i, r["choices"][0], flush=True)
        assert st == 200 and r["choices"][0]["tokens"] == want[:i] and r["choices"][0]["finish_reason"] == "stop"
        assert r["usage"]["completion_tokens"] == i
        # client stop ids are added to the model's
        st, r = post(srv.port, dict(prompt=[int(x) for x in prompt], max_tokens=24, temperature=0.0,
                                    stop_token_ids=[want[1]]))
        assert st == 200 and r["choices"][0]["tokens"] == want[:1] and r["choices"][0]["finish_reason"] == "stop"
        for body, word in ((dict(prompt=[1, 2], max_tokens=2 ** 32 + 16), "max_tokens"),
                           (dict(prompt=[1, 2], top_k=2 ** 32 + 1), "top_k"),
                           (dict(prompt=[1, 2], max_tokens=-1), "max_tokens")):
            st, r = post(srv.port, body)
            assert st == 400 and word in r["error"]["message"], (body, r)
        for seed in (-1, 2 ** 64 - 1):  # the same draws: -1 wraps to 2^64 - 1
            st, r = post(srv.port, dict(prompt=[int(x) for x in prompt], max_tokens=6, temperature=1.0, seed=seed))
            assert st == 200
            if seed == -1:
                first = r["choices"][0]["tokens"]
            else:
                assert r["choices"][0]["tokens"] == first
    finally:
        srv.close()
    # every finished request's result was released by the server: a fresh request gets a fresh id, and releasing it
    # leaves nothing held
    rid = eng.submit(prompt, max_tokens=3)
    eng.run()
    assert eng.release(rid) == 0
    with pytest.raises(mk_.MkError):
        eng.result(rid)
    eng.close()
    target.close()
