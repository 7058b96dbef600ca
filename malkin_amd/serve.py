"""Runs the HTTP API (include/malkin_server.h) over a GGUF model on one GPU until interrupted:

    python -m malkin_amd.serve --model m.gguf [--draft d.gguf] [--n-ctx 4096] [--parallel 1] [--port 8080]

The options are the reference's EngineOptions (engine.h:19-27: model, n_ctx, draft, n_draft, parallel) and its
serve(host, port); prompts and completions are token ids (no tokenizer in this build)."""
import argparse
import os
import signal
import threading

import malkin_amd as mk_


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--model", required=True)
    ap.add_argument("--draft", default="")
    ap.add_argument("--n-ctx", type=int, default=4096)
    ap.add_argument("--n-draft", type=int, default=0)
    ap.add_argument("--parallel", type=int, default=1)
    ap.add_argument("--host", default="127.0.0.1")
    ap.add_argument("--port", type=int, default=8080)
    ap.add_argument("--device", type=int, default=0)
    a = ap.parse_args()
    ctx = mk_.Context(a.device)
    target = mk_.Model(ctx, a.model, a.n_ctx, a.parallel)
    draft = mk_.Model(ctx, a.draft, a.n_ctx, a.parallel) if a.draft else None
    eng = mk_.Engine(target, draft, a.n_draft)
    srv = mk_.Server(eng, model_id=os.path.basename(a.model), host=a.host, port=a.port)
    print(f"malkin-mi355x: listening on http://{a.host}:{srv.port}", flush=True)
    done = threading.Event()
    signal.signal(signal.SIGINT, lambda *_: done.set())
    signal.signal(signal.SIGTERM, lambda *_: done.set())
    done.wait()
    srv.close()
    eng.close()
    if draft is not None:
        draft.close()
    target.close()
    ctx.close()


if __name__ == "__main__":
    main()
