"""The HTTP API's host half on the CPU (no device): routes, methods, errors and the JSON reader, through a server
started without an engine (include/malkin_server.h: 503 for completions)."""
import http.client
import json
import socket

import pytest

import malkin_amd as mk_


@pytest.fixture
def server():
    s = mk_.Server(None, model_id="tiny")
    yield s
    s.close()


def call(port, method, path, body=None, raw=None):
    c = http.client.HTTPConnection("127.0.0.1", port, timeout=30)
    data = raw if raw is not None else (json.dumps(body).encode() if body is not None else None)
    c.request(method, path, body=data, headers={"Content-Type": "application/json"} if data is not None else {})
    r = c.getresponse()
    out = r.status, r.read().decode()
    c.close()
    return out


def test_health_and_models(server):
    st, body = call(server.port, "GET", "/health")
    assert st == 200 and json.loads(body) == {"status": "ok"}
    st, body = call(server.port, "GET", "/v1/models?x=1")
    m = json.loads(body)
    assert st == 200 and m["object"] == "list" and m["data"][0]["id"] == "tiny"
    assert m["data"][0]["owned_by"] == "malkin" and m["data"][0]["context_length"] == 0


def test_errors(server):
    p = server.port
    st, body = call(p, "POST", "/health")
    assert st == 405
    st, body = call(p, "GET", "/nope")
    assert st == 404 and "error" in json.loads(body)
    for bad in (b"{", b'{"a":1} x', b'{"a":"\\q"}', b'{"a":"\\ud800"}', b"[1,]", b'{"a" 1}', b"\x01"):
        st, body = call(p, "POST", "/v1/completions", raw=bad)
        e = json.loads(body)["error"]
        assert st == 400 and e["type"] == "invalid_request_error" and e["message"].startswith("bad json"), bad
    st, body = call(p, "POST", "/v1/completions", raw=b"[1, 2]")
    assert st == 400 and "object" in json.loads(body)["error"]["message"]
    st, body = call(p, "POST", "/v1/completions", {"prompt": [1, 2]})
    assert st == 503 and json.loads(body)["error"]["type"] == "server_error"
    st, body = call(p, "POST", "/v1/chat/completions", {"messages": []})
    assert st == 400 and "tokenizer" in json.loads(body)["error"]["message"]
    # a malformed request line and an oversized body
    with socket.create_connection(("127.0.0.1", p), timeout=30) as s:
        s.sendall(b"GARBAGE\r\n\r\n")
        assert s.recv(100).startswith(b"HTTP/1.1 400")
    with socket.create_connection(("127.0.0.1", p), timeout=30) as s:
        s.sendall(b"POST /v1/completions HTTP/1.1\r\nContent-Length: 999999999999\r\n\r\n")
        assert s.recv(100).startswith(b"HTTP/1.1 413")


def test_json_reader_accepts_the_grammar(server):
    """Valid documents reach the route (503 = parsed, no engine): escapes, surrogate pairs, exponents, nesting."""
    for good in (b'{"prompt":[1,2,3],"x":"\\u00e9\\ud83d\\ude00\\n","y":-1.5e-3,"z":[true,false,null,{}]}',
                 b' { "prompt" : [ ] } ', b'{"seed":18446744073709551615}'):
        st, body = call(server.port, "POST", "/v1/completions", raw=good)
        assert st == 503, (good, body)


def test_stop_is_clean_with_connections_open():
    s = mk_.Server(None)
    conn = socket.create_connection(("127.0.0.1", s.port), timeout=30)
    conn.sendall(b"GET /health HTTP/1.1\r\n\r\n")
    assert conn.recv(100).startswith(b"HTTP/1.1 200")
    s.close()
    conn.close()
    with pytest.raises(OSError):
        socket.create_connection(("127.0.0.1", s.port), timeout=5).close()
