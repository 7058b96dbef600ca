"""Benchmark: the north-star workload of BASELINE.json on one MI355X.

Workload (one "step"): a random-init Qwen3-8B-architecture model in Q8_0 (36 layers, hidden 4096, 32/8 heads,
head_dim 128, FFN 12288, vocab 151936, untied LM head), ctx 4096, batch 1 — a 512-token prompt evaluated in two
256-token forwards (the reference engine's kMaxBatch chunks), then greedy decoding to 128 generated tokens (the first
from the prompt's logits, 127 decode forwards), as `malkin bench` does (main.cpp:126-143).

value = (512 + 128) tokens / wall time of the step, inputs (weights, prompt) resident in HBM before the timed region.
The JSON line also carries pp512 and tg128 rates, the live roofline of the dominant kernel (the Q8_0 decode GEMV,
timed with HIP events on the library's stream) and the reference's own AVX-512 path timed on this host's cores on a
bounded sample of the same workload (cpu_baseline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "pp512 + tg128 tokens/s, Qwen3-8B-shape Q8_0, 1 GPU; % of HBM/MFMA peak"
HBM_PEAK_GBS = 8000.0
N_PROMPT, N_GEN, N_CTX = 512, 128, 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prompt_ids(n, vocab):
    # `malkin bench` uses fixed ids 1000 + (i * 7919) % 20000 (main.cpp:128-129)
    return np.array([1000 + (i * 7919) % 20000 for i in range(n)], dtype=np.int32) % vocab


def model_file(preset, seed):
    from malkin_amd import synth
    cfg = synth.make_config(preset, synth.Q8_0, seed=seed)
    d = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    st = os.statvfs(d)
    if st.f_bavail * st.f_frsize < synth.file_bytes(cfg) * 1.1:
        d = tempfile.gettempdir()
    path = os.path.join(d, f"malkin_bench_{preset}_q8_0_s{seed}_{os.getpid()}.gguf")
    t0 = time.time()
    synth.write_gguf(path, cfg, threads=min(16, os.cpu_count() or 1))
    log(f"[bench] wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.time() - t0:.1f} s")
    return path, cfg


def gemv_roofline(ctx, model, cfg, reps=3):
    """Live roofline of the dominant kernel: the Q8_0 decode GEMV (n = 1) over one decode step's 144 layer matmuls
    (q|k|v, attn_output, gate|up, down of 36 layers: 7.0 GB, far beyond the 256 MB Infinity Cache), timed with HIP
    events on the library stream. Algorithmic bytes per launch = GGUF bytes of the weight (34 B per 32 weights) + the
    BlockQ8 input (40 B per 32) + the f32 output."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    E, F = cfg["n_embd"], cfg["n_ff"]
    xin = ctx.alloc(max(E, F) // 32 * 40)
    rng = np.random.default_rng(0)
    xb = np.zeros(max(E, F) // 32, dtype=mk.BLOCK_Q8)
    xb["d"] = rng.uniform(0.01, 0.05, xb.size)
    xb["qs"] = rng.integers(-127, 128, (xb.size, 32))
    xb["s"][:, 0] = xb["qs"][:, :16].sum(1)
    xb["s"][:, 1] = xb["qs"][:, 16:].sum(1)
    xin.upload(xb)
    yout = ctx.alloc(2 * F * 4)
    ws = [model.weight(l, w) for l in range(cfg["n_layer"]) for w in range(4)]
    algo = sum(w.rows * w.cols // 32 * 34 + w.cols // 32 * 40 + w.rows * 4 for w in ws)
    for w in ws:  # warm
        mk.check(L.mk_matmul(ctx.h, ctypes.byref(w), xin.ptr, 1, yout.ptr, w.rows, 0))
    ctx.sync()
    best = None
    for _ in range(reps):
        ctx.timer_start()
        for w in ws:
            mk.check(L.mk_matmul(ctx.h, ctypes.byref(w), xin.ptr, 1, yout.ptr, w.rows, 0))
        ms = ctx.timer_stop()
        best = ms if best is None else min(best, ms)
    launches = len(ws)
    per_launch_s = best / 1e3 / launches
    achieved = algo / launches / per_launch_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": "k_gemv<Q8_0, n=1> (decode GEMV, 144 launches per token)",
            "bytes_per_launch": int(algo / launches), "us_per_launch": round(per_launch_s * 1e6, 2)}


def cpu_baseline(path, vocab, budget_s=30.0):
    """The reference's own AVX-512 path (oracle/_ref, compiled from its sources), timed on this host's cores with
    OMP threads = physical cores (the reference's default, engine.cpp:104-109). Sample: the pp512 prompt in two
    256-token forwards, then decode forwards until about budget_s of CPU work; tg from the measured decode rate."""
    from oracle import bind
    if not bind.ref_available():
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref not built on this tree"}
    ref = bind.Ref()
    if not ref.cpu_ok():
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference",
                "sample": f"host CPU ({ref.cpu_model()}) lacks AVX-512 VNNI/BF16"}
    cores = ref.physical_cores()
    ref.set_threads(cores)
    t0 = time.time()
    m = ref.model(path, N_PROMPT + N_GEN, 1)
    load_s = time.time() - t0
    p = prompt_ids(N_PROMPT, vocab)
    t0 = time.time()
    m.forward(p[:256], 0)
    logits = m.forward(p[256:], 256)
    pp_s = time.time() - t0
    tok = int(np.argmax(logits[0]))
    t0 = time.time()
    n_dec = 0
    while n_dec < N_GEN - 1 and (time.time() - t0) < max(1.0, budget_s - pp_s):
        logits = m.forward(np.array([tok], np.int32), N_PROMPT + n_dec)
        tok = int(np.argmax(logits[0]))
        n_dec += 1
    dec_s = time.time() - t0
    m.close()
    per_tok = dec_s / n_dec
    step_s = pp_s + per_tok * (N_GEN - 1)
    return {"value": round((N_PROMPT + N_GEN) / step_s, 3), "unit": "tokens/s", "cores": cores, "kind": "reference",
            "sample": f"pp512 (2 x 256-token forwards) + {n_dec} of the 127 decode forwards, the rest extrapolated "
                      f"at the measured rate; {ref.cpu_model()}, {cores} threads; panel packing {load_s:.1f} s "
                      f"untimed",
            "pp512_tok_s": round(N_PROMPT / pp_s, 2), "tg_tok_s": round(1.0 / per_tok, 3)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--preset", default="qwen3-8b")
    ap.add_argument("--no-graph", action="store_true",
                    help="decode with direct launches instead of the replayed HIP graph (for tracers that do not "
                         "follow graph launches); same kernels")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)

    import malkin_amd as mk
    mk.load()
    path, _ = model_file(args.preset, seed=1)
    try:
        ctx = mk.Context(0)
        t0 = time.time()
        model = mk.Model(ctx, path, N_CTX, 1)
        log(f"[bench] model on {ctx.device_name}: {model.weight_bytes / 1e9:.2f} GB packed, "
            f"load {time.time() - t0:.1f} s")
        cfg = model.cfg
        prompt = prompt_ids(N_PROMPT, cfg["n_vocab"])
        for i in range(args.warmup):
            toks, st = model.generate(prompt, N_GEN, use_graph=not args.no_graph)
            log(f"[bench] warmup {i}: prefill {st['prefill_ms']:.1f} ms, decode {st['decode_ms']:.1f} ms")
        ctx.sync()
        pre, dec = [], []
        t_start = time.perf_counter()
        for i in range(args.steps):
            toks, st = model.generate(prompt, N_GEN, use_graph=not args.no_graph)
            pre.append(st["prefill_ms"])
            dec.append(st["decode_ms"])
            log(f"[bench] step {i}: prefill {st['prefill_ms']:.1f} ms, decode {st['decode_ms']:.1f} ms")
        ctx.sync()
        wall = time.perf_counter() - t_start
        ms_step = wall * 1e3 / args.steps
        roof = gemv_roofline(ctx, model, cfg)
        log(f"[bench] decode GEMV: {roof['achieved']} GB/s ({roof['us_per_launch']} us per launch)")
        cpu = None if args.no_cpu_baseline else cpu_baseline(path, cfg["n_vocab"])
        model.close()
        ctx.close()
    finally:
        if os.path.exists(path):
            os.remove(path)

    pp_ms, dec_ms = float(np.median(pre)), float(np.median(dec))
    line = {
        "metric": METRIC,
        "value": round((N_PROMPT + N_GEN) * 1e3 / ms_step, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint8->int32, f32 (Q8_0)",
        "data": "synthetic: random-init weights N(0, 0.02) quantized to Q8_0, fixed prompt ids",
        "config": {"workload": "qwen3-8b-q8_0 pp512+tg128, batch 1, ctx 4096, greedy", "prompt_tokens": N_PROMPT,
                   "gen_tokens": N_GEN, "decode_forwards": N_GEN - 1, "parallelism": "none (1 GPU)"},
        "pp512_tok_s": round(N_PROMPT * 1e3 / pp_ms, 1),
        "tg128_tok_s": round((N_GEN - 1) * 1e3 / dec_ms, 2),
        "decode_ms_per_token": round(dec_ms / (N_GEN - 1), 4),
        "decode_hbm_frac": round(model_bytes_per_token(cfg) / (dec_ms / (N_GEN - 1) / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": roof,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def model_bytes_per_token(cfg):
    """Algorithmic bytes of one decode token: GGUF bytes of every matmul weight read (incl. the LM head)."""
    E, F, H, KV, D, V, L = (cfg[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab",
                                              "n_layer"))
    per_layer = ((H + 2 * KV) * D * E + E * H * D + 2 * F * E + E * F) // 32 * 34
    return per_layer * L + V * E // 32 * 34


if __name__ == "__main__":
    main()
