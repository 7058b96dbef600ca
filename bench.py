"""Benchmark: the north-star workload of BASELINE.json on one MI355X.

Workload (one "step"): a random-init Qwen3-8B-architecture model in Q8_0 (36 layers, hidden 4096, 32/8 heads,
head_dim 128, FFN 12288, vocab 151936, untied LM head), ctx 4096, batch 1 — a 512-token prompt evaluated in one
512-token forward (the reference's engine takes 256 per forward, engine.cpp:381-393; every token's results are the
same either way), then greedy decoding to 128 generated tokens (the first from the prompt's logits, 127 decode
forwards), as `malkin bench` does (main.cpp:126-143).

value = (512 + 128) tokens / wall time of the step, inputs (weights, prompt) resident in HBM before the timed region.
The JSON line also carries pp512 and tg128 rates, pp512 in the reference engine's protocol (two 256-token forwards,
pp512_2x256_tok_s, the cpu_baseline leg's protocol), the prefill's fraction of the int8 MFMA peak, the live roofline of
the dominant kernel (the Q8_0 decode GEMV, timed with HIP events on the library's stream; its HBM traffic from the
committed counter summary), the kernel-level configurations 1 and 2 of BASELINE.json (kernel_configs), and the
reference's own AVX-512 path timed on this host's cores on a bounded sample of the same workload (cpu_baseline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-kernel-configs]
    python bench.py --probe traffic     # launch sequence for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
    python bench.py --probe gemm        # the prefill GEMM shapes, for counter passes
    python bench.py --probe kquant      # config 2's Q4_K shapes at n = 1, 4, 8, for counter passes
    python bench.py --probe rows        # the pp512 forward's prefill attention, for counter passes
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


def model_file(preset, seed, wtype=None, mix=None):
    from malkin_amd import synth
    wtype = synth.Q8_0 if wtype is None else wtype
    mix = synth.MIX_UNIFORM if mix is None else mix
    cfg = synth.make_config(preset, wtype, mix=mix, seed=seed)
    d = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    st = os.statvfs(d)
    if st.f_bavail * st.f_frsize < synth.file_bytes(cfg) * 1.1:
        d = tempfile.gettempdir()
    path = os.path.join(d, f"malkin_bench_{preset}_t{wtype}_m{mix}_s{seed}_{os.getpid()}.gguf")
    t0 = time.time()
    synth.write_gguf(path, cfg, threads=min(16, os.cpu_count() or 1))
    log(f"[bench] wrote {path} ({os.path.getsize(path) / 1e9:.2f} GB) in {time.time() - t0:.1f} s")
    return path, cfg


def gemv_roofline(ctx, model, cfg, reps=3):
    """Live roofline of the dominant kernel: the decode GEMV family (n = 1) exactly as the timed decode launches it
    (Model::run): per layer q|k|v with rmsnorm + quantization in its prologue, attn_output from the fp32 attention
    rows with the residual add in its epilogue, gate|up with rmsnorm + quantization in the prologue and silu(gate)*up
    in the epilogue, down from the fp32 SwiGLU rows with the residual add; 144 launches over the 36 layers (7.0 GB,
    far beyond the 256 MB Infinity Cache), timed with HIP events on the library stream. Algorithmic bytes per launch
    = GGUF bytes of the weight (34 B per 32 weights) + the fp32 input row (+ norm weights) + the fp32 output (read
    and written where the epilogue accumulates)."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    E, F, H, D = cfg["n_embd"], cfg["n_ff"], cfg["n_head"], cfg["head_dim"]
    eps = ctypes.c_float(cfg["rms_eps"])
    rng = np.random.default_rng(0)
    x = ctx.to_device(rng.standard_normal(E).astype(np.float32))
    att = ctx.to_device(rng.standard_normal(H * D).astype(np.float32))
    norm = ctx.to_device(np.ones(E, np.float32))
    qkv = ctx.alloc((H + 2 * cfg["n_head_kv"]) * D * 4)
    gu = ctx.to_device(rng.standard_normal(F).astype(np.float32))
    res = ctx.to_device(np.zeros(E, np.float32))
    calls, algo = [], 0
    for layer in range(cfg["n_layer"]):
        wq, wo, wg, wd = (model.weight(layer, i) for i in range(4))
        calls += [(wq, x, E, norm, qkv, wq.rows, 0, 0), (wo, att, H * D, None, res, E, 1, 0),
                  (wg, x, E, norm, gu, F, 0, 1), (wd, gu, F, None, res, E, 1, 0)]
        for w, _, k, nw, _, rows_out, acc, silu in calls[-4:]:
            algo += w.rows * w.cols // 32 * 34 + k * 4 + (k * 4 if nw is not None else 0) + rows_out * 4 * (1 + acc)

    def run():
        for w, xin, xs, nw, y, ys, acc, silu in calls:
            mk.check(L.mk_matmul_f32(ctx.h, ctypes.byref(w), xin.ptr, xs, nw.ptr if nw is not None else None, eps, 1,
                                     y.ptr, ys, acc, silu))

    run()  # warm
    ctx.sync()
    best = None
    for _ in range(reps):
        ctx.timer_start()
        run()
        ms = ctx.timer_stop()
        best = ms if best is None else min(best, ms)
    for b in (x, att, norm, qkv, gu, res):
        b.free()
    launches = len(calls)
    per_launch_s = best / 1e3 / launches
    achieved = algo / launches / per_launch_s / 1e9
    return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": roofline_traffic(),
            "kernel": "k_gemv<Q8_0, n=1> with the decode's fused prologues/epilogues (q|k|v norm, attn_output "
                      "residual, gate|up norm + silu, down residual; 144 launches per token)",
            "bytes_per_launch": int(algo / launches), "us_per_launch": round(per_launch_s * 1e6, 2)}


# GGUF block geometry: (values per block, bytes per block, byte offsets of the f16 scales).
_BLOCKS = {8: (32, 34, (0,)), 12: (256, 144, (0, 2)), 14: (256, 210, (208,))}
INT8_PEAK_TOPS = 5000.0


def random_weight(rng, t, rows, cols):
    """GGUF rows of type t drawn as BASELINE.json states: entries N(0, 0.02), quantized by the synthetic model
    writer's quantizer (the reference ships none), in slabs of 1024 rows."""
    from malkin_amd import synth
    out = []
    for r in range(0, rows, 1024):
        n = min(1024, rows - r)
        out.append(synth.quantize_rows(t, rng.normal(0.0, 0.02, (n, cols)).astype(np.float32)))
    return np.concatenate(out)


def pack_copies(ctx, t, host_rows, rows, cols, copies):
    """`copies` packed device copies of one weight (distinct addresses, so rotating them defeats the 256 MB cache)."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    src = ctx.to_device(host_rows)
    out = []
    for _ in range(copies):
        b = ctx.alloc(L.mk_packed_bytes(t, rows, cols))
        mk.check(L.mk_pack_weight(ctx.h, t, src.ptr, host_rows.shape[1], rows, cols, b.ptr))
        out.append((b, mk.MkWeight(t, 1, rows, cols, b.p)))
    src.free()
    return out


def random_acts(ctx, rng, n, k):
    """n rows of N(0, 1) activations, quantized to BlockQ8 on the device (quantize_acts)."""
    import malkin_amd as mk
    x = ctx.to_device(rng.standard_normal((n, k)).astype(np.float32))
    xq = ctx.alloc(n * (k // 32) * 40)
    mk.check(mk.load().mk_quantize_q8(ctx.h, x.ptr, n, k, xq.ptr))
    x.free()
    return xq


def time_matmuls(ctx, ws, xq, n, y, reps):
    """Average time (s) of one mk_matmul launch, cycling through the weights ws, HIP events on the library stream."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    for _, w in ws:
        mk.check(L.mk_matmul(ctx.h, ctypes.byref(w), xq.ptr, n, y.ptr, w.rows, 0))
    ctx.sync()
    ctx.timer_start()
    for i in range(reps):
        w = ws[i % len(ws)][1]
        mk.check(L.mk_matmul(ctx.h, ctypes.byref(w), xq.ptr, n, y.ptr, w.rows, 0))
    return ctx.timer_stop() / 1e3 / reps


def kernel_configs(ctx):
    """The kernel-level configurations of BASELINE.json:
    config 1: one Q8_0 GEMM, W 9728x2560, X 512x2560 (int8 MFMA prefill kernel): time, TOPS, fraction of int8 peak;
    config 2: decode GEMV, Qwen3-14B FFN shapes (gate/up 5120->17408, down 17408->5120) in Q4_K and Q6_K at n = 1, 4,
    8, cycling through 8 packed copies of each matrix (more than the 256 MB Infinity Cache holds): GB/s of algorithmic
    bytes (GGUF weight bytes + BlockQ8 input + f32 output) and fraction of the 8 TB/s HBM peak."""
    import malkin_amd as mk
    rng = np.random.default_rng(7)
    out = {}
    rows, cols, n = 9728, 2560, 512
    ws = pack_copies(ctx, mk.Q8_0, random_weight(rng, mk.Q8_0, rows, cols), rows, cols, 1)
    xq, y = random_acts(ctx, rng, n, cols), ctx.alloc(n * rows * 4)
    t = time_matmuls(ctx, ws, xq, n, y, 20)
    ops = 2.0 * n * rows * cols
    out["gemm_q8_0_9728x2560_n512"] = {"us": round(t * 1e6, 2), "tops": round(ops / t / 1e12, 1),
                                       "mfma_frac": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4)}
    for b, _w in ws:
        b.free()
    xq.free()
    y.free()
    for t_name, t in (("q4_k", mk.Q4_K), ("q6_k", mk.Q6_K)):
        for rows, cols in ((17408, 5120), (5120, 17408)):
            qk, bs, _ = _BLOCKS[t]
            wbytes = rows * (cols // qk) * bs
            ws = pack_copies(ctx, t, random_weight(rng, t, rows, cols), rows, cols, 8)
            y = ctx.alloc(8 * rows * 4)
            for n in (1, 4, 8):
                xq = random_acts(ctx, rng, n, cols)
                sec = time_matmuls(ctx, ws, xq, n, y, 32)
                gbs = (wbytes + n * (cols // 32) * 40 + n * rows * 4) / sec / 1e9
                out[f"gemv_{t_name}_{rows}x{cols}_n{n}"] = {"us": round(sec * 1e6, 2), "gbs": round(gbs, 1),
                                                           "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)}
                xq.free()
            y.free()
            for b, _w in ws:
                b.free()
    return out


def decode_probe():
    """Launch sequence for the instruction / wait / LDS counters of one decode layer's kernels (run under rocprofv3
    --pmc with one counter group per pass): the fused decode attention of the Qwen3-8B shape (32 query heads over 8
    KV heads, head_dim 128) at 600 keys with its QK-norm / RoPE / KV write and BlockQ8 output (mk_attention_decode_q8),
    then the four decode GEMVs as the decode launches them (q|k|v with the norm prologue, attn_output accumulating,
    gate|up with the norm prologue and SiLU epilogue, down accumulating), each 4 times."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    ctx = mk.Context(0)
    rng = np.random.default_rng(5)
    eps = ctypes.c_float(1e-6)
    D, H, KV, n_ctx, pos = 128, 32, 8, 1024, 599
    QKV = (H + 2 * KV) * D
    qkv = ctx.to_device(rng.standard_normal(QKV).astype(np.float32))
    norms = ctx.to_device(rng.uniform(0.5, 1.5, 2 * D).astype(np.float32))
    ang = np.arange(n_ctx, dtype=np.float32)[:, None] * np.float32(1e-3) * (np.arange(D // 2, dtype=np.float32) + 1)
    cos_t, sin_t = ctx.to_device(np.cos(ang).astype(np.float32)), ctx.to_device(np.sin(ang).astype(np.float32))
    k8 = ctx.to_device(rng.integers(-127, 128, (1, KV, n_ctx, D), dtype=np.int8))
    v8 = ctx.to_device(rng.integers(-127, 128, (1, KV, n_ctx, D), dtype=np.int8))
    ks = ctx.to_device(rng.uniform(0.001, 0.05, (1, KV, n_ctx)).astype(np.float32))
    vs = ctx.to_device(rng.uniform(0.001, 0.05, (1, KV, n_ctx)).astype(np.float32))
    kv = mk.MkKvCache(k8.ptr, v8.ptr, ks.ptr, vs.ptr, 1, 1, KV, D, n_ctx)
    meta = {nm: ctx.to_device(np.array([v], np.int32)) for nm, v in (("rpos", pos), ("seq", 0), ("kv_row", pos),
                                                                       ("n_keys", pos + 1))}
    out, xq = ctx.alloc(H * D * 4), ctx.alloc(H * D // 32 * 40)
    ctx.sync()
    for i in range(4):
        mk.check(L.mk_attention_decode_q8(ctx.h, qkv.ptr, QKV, 1, H, norms.ptr, norms.offset(D * 4), eps, cos_t.ptr,
                                          sin_t.ptr, meta["rpos"].ptr, meta["seq"].ptr, meta["kv_row"].ptr,
                                          meta["n_keys"].ptr, ctypes.byref(kv), 0, out.ptr, H * D, pos + 1, xq.ptr))
    ctx.sync()
    log(f"[probe] k_attention_dec: {H} heads over {KV} KV heads, head_dim {D}, {pos + 1} keys: 4 launches")
    for rows, cols, norm, acc, silu in ((6144, 4096, 1, 0, 0), (4096, 4096, 0, 1, 0), (24576, 4096, 1, 0, 1),
                                        (4096, 12288, 0, 1, 0)):
        ws = pack_copies(ctx, mk.Q8_0, random_weight(rng, mk.Q8_0, rows, cols), rows, cols, 2)
        x = ctx.to_device(rng.standard_normal(cols).astype(np.float32))
        nw = ctx.to_device(np.ones(cols, np.float32)) if norm else None
        out_rows = rows // 2 if silu else rows
        y = ctx.to_device(np.zeros(out_rows, np.float32))
        ctx.sync()
        for i in range(4):
            mk.check(L.mk_matmul_f32(ctx.h, ctypes.byref(ws[i % 2][1]), x.ptr, cols, nw.ptr if nw else None, eps, 1,
                                     y.ptr, out_rows, acc, silu))
        ctx.sync()
        log(f"[probe] k_gemv Q8_0 {rows}x{cols} n=1 (norm {norm}, accumulate {acc}, silu {silu}): 4 launches")
        for b, _w in ws:
            b.free()
        for b in (x, nw, y):
            if b is not None:
                b.free()
    ctx.close()


def traffic_probe():
    """Launch sequence for the HBM-traffic counters of the roofline kernel (run under rocprofv3 --pmc FETCH_SIZE, then
    WRITE_SIZE): the four decode GEMV variants of the Qwen3-8B layer as the decode launches them (q|k|v 6144x4096 with
    the norm prologue, attn_output 4096x4096 accumulating, gate|up 24576x4096 with the norm prologue and SiLU epilogue,
    down 4096x12288 accumulating) at n = 1, each launched 4 times over 2 packed copies, then one plain 256 MiB
    device-to-device copy (the counter scale: it reads and writes exactly 256 MiB)."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    ctx = mk.Context(0)
    rng = np.random.default_rng(3)
    eps = ctypes.c_float(1e-6)
    for rows, cols, norm, acc, silu in ((6144, 4096, 1, 0, 0), (4096, 4096, 0, 1, 0), (24576, 4096, 1, 0, 1),
                                        (4096, 12288, 0, 1, 0)):
        ws = pack_copies(ctx, mk.Q8_0, random_weight(rng, mk.Q8_0, rows, cols), rows, cols, 2)
        x = ctx.to_device(rng.standard_normal(cols).astype(np.float32))
        nw = ctx.to_device(np.ones(cols, np.float32)) if norm else None
        out_rows = rows // 2 if silu else rows
        y = ctx.to_device(np.zeros(out_rows, np.float32))
        ctx.sync()
        for i in range(4):
            w = ws[i % 2][1]
            mk.check(L.mk_matmul_f32(ctx.h, ctypes.byref(w), x.ptr, cols, nw.ptr if nw else None, eps, 1, y.ptr,
                                     out_rows, acc, silu))
        ctx.sync()
        algo = rows * cols // 32 * 34 + cols * 4 * (2 if norm else 1) + out_rows * 4 * (1 + acc)
        log(f"[probe] k_gemv Q8_0 {rows}x{cols} n=1 (norm {norm}, accumulate {acc}, silu {silu}): 4 launches, "
            f"algorithmic bytes {algo}")
        for b, _w in ws:
            b.free()
        for b in (x, nw, y):
            if b is not None:
                b.free()
    hip = ctypes.CDLL("libamdhip64.so")
    nbytes = 256 << 20
    a, b = ctx.alloc(nbytes), ctx.alloc(nbytes)
    ctx.sync()
    rc = hip.hipMemcpy(ctypes.c_void_p(b.p), ctypes.c_void_p(a.p), ctypes.c_size_t(nbytes), 3)
    hip.hipDeviceSynchronize()
    log(f"[probe] hipMemcpy device-to-device {nbytes} bytes (rc {rc})")
    ctx.close()


def gemm_probe():
    """Launch sequence for the prefill GEMM's counters (rocprofv3 --pmc): config 1 (Q8_0 9728x2560, n = 512) 8 times,
    then the Qwen3-8B shapes of the pp512 forward (q|k|v 6144x4096, attn_output 4096x4096, gate|up 24576x4096, down
    4096x12288, n = 512) 4 times each, from BlockQ8 activations."""
    import malkin_amd as mk
    ctx = mk.Context(0)
    rng = np.random.default_rng(5)
    for rows, cols, n, reps in ((9728, 2560, 512, 8), (6144, 4096, 512, 4), (4096, 4096, 512, 4),
                                (24576, 4096, 512, 4), (4096, 12288, 512, 4)):
        ws = pack_copies(ctx, mk.Q8_0, random_weight(rng, mk.Q8_0, rows, cols), rows, cols, 1)
        xq, y = random_acts(ctx, rng, n, cols), ctx.alloc(n * rows * 4)
        ctx.sync()
        sec = time_matmuls(ctx, ws, xq, n, y, reps)
        log(f"[probe] k_gemm_q8_0 {rows}x{cols} n={n}: {reps} launches, {sec * 1e6:.2f} us each, "
            f"{2.0 * n * rows * cols / sec / 1e12:.1f} TOPS")
        for b, _w in ws:
            b.free()
        xq.free()
        y.free()
    ctx.close()


def kquant_probe():
    """Launch sequence for the short-batch K-quant counters (rocprofv3 --pmc / --kernel-trace): config 2's Q4_K shapes
    (gate/up 17408x5120, down 5120x17408) at n = 1, 4, 8, each 8 launches over 4 packed copies, from BlockQ8
    activations."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    ctx = mk.Context(0)
    rng = np.random.default_rng(0)
    y = ctx.alloc(8 * 17408 * 4)
    for rows, cols in ((17408, 5120), (5120, 17408)):
        ws = pack_copies(ctx, mk.Q4_K, random_weight(rng, mk.Q4_K, rows, cols), rows, cols, 4)
        for n in (1, 4, 8):
            xq = random_acts(ctx, rng, n, cols)
            for i in range(8):
                mk.check(L.mk_matmul(ctx.h, ctypes.byref(ws[i % 4][1]), xq.ptr, n, y.ptr, rows, 0))
            ctx.sync()
            log(f"[probe] Q4_K {rows}x{cols} n={n}: 8 launches")
            xq.free()
        for b, _w in ws:
            b.free()
    y.free()
    ctx.close()


def roofline_traffic():
    """HBM bytes per launch of the roofline kernel, from the committed counter summary (profiles/), or None."""
    f = os.path.join(ROOT, "profiles", "k_gemv_q8_0_decode_n1_hbm_traffic.md")
    if not os.path.exists(f):
        return None
    for line in open(f):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def cpu_baseline(path, prompt, gpu_tokens, budget_s=30.0):
    """The reference's own AVX-512 path (oracle/_ref, compiled from its sources), timed on this host's cores with
    OMP threads = physical cores (the reference's default, engine.cpp:104-109). Sample: the 512-token prompt in two
    256-token forwards, then greedy decode forwards until about budget_s of CPU work; tg from the measured decode rate.
    Its greedy ids are compared with the device's stream on the same model and prompt (tokens_match)."""
    from oracle import bind
    if not bind.ref_available():
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference",
                "sample": "oracle/_ref not built on this tree", "tokens_match": None}
    ref = bind.Ref()
    if not ref.cpu_ok():
        return {"value": None, "unit": "tokens/s", "cores": 0, "kind": "reference",
                "sample": f"host CPU ({ref.cpu_model()}) lacks AVX-512 VNNI/BF16", "tokens_match": None}
    cores = ref.physical_cores()
    ref.set_threads(cores)
    n_prompt, n_gen = len(prompt), len(gpu_tokens)
    t0 = time.time()
    m = ref.model(path, n_prompt + n_gen, 1)
    load_s = time.time() - t0
    t0 = time.time()
    for i in range(0, n_prompt, 256):
        logits = m.forward(prompt[i:i + 256], i)
    pp_s = time.time() - t0
    ids = [int(np.argmax(logits[0]))]
    t0 = time.time()
    n_dec = 0
    while n_dec < n_gen - 1 and (time.time() - t0) < max(1.0, budget_s - pp_s):
        logits = m.forward(np.array([ids[-1]], np.int32), n_prompt + n_dec)
        ids.append(int(np.argmax(logits[0])))
        n_dec += 1
    dec_s = time.time() - t0
    m.close()
    per_tok = dec_s / max(n_dec, 1)
    step_s = pp_s + per_tok * (n_gen - 1)
    match = [int(a) for a in gpu_tokens[:len(ids)]] == ids
    return {"value": round((n_prompt + n_gen) / step_s, 3), "unit": "tokens/s", "cores": cores, "kind": "reference",
            "sample": f"pp{n_prompt} ({(n_prompt + 255) // 256} x 256-token forwards) + {n_dec} of the {n_gen - 1} "
                      f"decode forwards, the rest extrapolated at the measured rate; {ref.cpu_model()}, {cores} "
                      f"threads; panel packing {load_s:.1f} s untimed",
            "pp_tok_s": round(n_prompt / pp_s, 2), "tg_tok_s": round(1.0 / per_tok, 3),
            "tokens_compared": len(ids), "tokens_match": match}


def config3(ctx, reps=3, with_cpu=True, use_graph=True):
    """random-init Qwen3-4B architecture in Q8_0 (36 layers, hidden 2560, 32/8 heads, head_dim 128,
    FFN 9728 SwiGLU, vocab 151936, tied embeddings; synthetic seed 31), a prompt of 512 uniform-random ids (numpy
    seed 303), 128 greedy tokens, ctx 4096: pp512 + tg128 on the device with the same protocol as the main line, its
    HBM / int8-MFMA fractions, and the reference's AVX-512 path on the same model and prompt (greedy ids compared)."""
    import malkin_amd as mk
    path, _ = model_file("qwen3-4b", seed=31)
    try:
        m = mk.Model(ctx, path, N_CTX, 1)
        cfg = m.cfg
        prompt = np.random.default_rng(303).integers(0, cfg["n_vocab"], N_PROMPT).astype(np.int32)
        m.generate(prompt, N_GEN, use_graph=use_graph)
        ctx.sync()
        pre, dec = [], []
        t0 = time.perf_counter()
        for _ in range(reps):
            toks, st = m.generate(prompt, N_GEN, use_graph=use_graph)
            pre.append(st["prefill_ms"])
            dec.append(st["decode_ms"])
        ctx.sync()
        ms_step = (time.perf_counter() - t0) * 1e3 / reps
        m.close()
        pp_ms, dec_ms = float(np.median(pre)), float(np.median(dec))
        out = {"workload": "qwen3-4b-q8_0 pp512+tg128, 512 uniform-random prompt ids, batch 1, ctx 4096, greedy",
               "tokens_per_s": round((N_PROMPT + N_GEN) * 1e3 / ms_step, 2), "ms_per_step": round(ms_step, 3),
               "pp512_tok_s": round(N_PROMPT * 1e3 / pp_ms, 1), "tg128_tok_s": round((N_GEN - 1) * 1e3 / dec_ms, 2),
               "decode_ms_per_token": round(dec_ms / (N_GEN - 1), 4),
               "decode_hbm_frac": round(model_bytes_per_token(cfg) / (dec_ms / (N_GEN - 1) / 1e3) / 1e9 / HBM_PEAK_GBS,
                                        4),
               "pp512_mfma_frac": round(prefill_ops(cfg) / (pp_ms / 1e3) / 1e12 / INT8_PEAK_TOPS, 4)}
        if with_cpu:
            out["cpu_baseline"] = cpu_baseline(path, prompt, toks, budget_s=15.0)
        return out
    finally:
        if os.path.exists(path):
            os.remove(path)


def config4(ctx, path):
    """the Qwen3-8B Q8_0 model, 8 concurrent sequences with random-id prompts of 256..1024 tokens,
    128 greedy tokens each, continuous batching on the device engine (one batched forward per step: decode rows of
    every decoding sequence plus prompt chunks up to 256 tokens), KV cache ctx 4096 per sequence."""
    import malkin_amd as mk
    rng = np.random.default_rng(4)
    m = mk.Model(ctx, path, N_CTX, 8)
    try:
        V = m.cfg["n_vocab"]
        prompts = [rng.integers(0, V, size=int(L)).astype(np.int32) for L in rng.integers(256, 1025, size=8)]
        warm = mk.Engine(m)
        warm.submit(prompts[0][:64], 4)
        warm.run()
        warm.close()
        e = mk.Engine(m)
        ctx.sync()
        t0 = time.perf_counter()
        ids = [e.submit(p, 128) for p in prompts]
        steps = 0
        while e.step() > 0:
            steps += 1
        ctx.sync()
        wall = time.perf_counter() - t0
        infos = [e.result(i)[1] for i in ids]
        e.close()
    finally:
        m.close()
    n_prompt = int(sum(len(p) for p in prompts))
    n_gen = int(sum(i["completion_tokens"] for i in infos))
    return {"workload": "qwen3-8b-q8_0, 8 sequences, prompts 256..1024 (random ids), 128 greedy tokens each, "
                        "continuous batching, ctx 4096",
            "prompt_tokens": n_prompt, "gen_tokens": n_gen, "engine_steps": steps + 1, "wall_s": round(wall, 3),
            "tokens_per_s": round((n_prompt + n_gen) / wall, 1), "gen_tokens_per_s": round(n_gen / wall, 1),
            "mean_prefill_ms": round(float(np.mean([i["prefill_ms"] for i in infos])), 1),
            "mean_decode_ms": round(float(np.mean([i["decode_ms"] for i in infos])), 1)}


def tree_nodes(ids, P):
    """The engine's 17-node tree over a P-token prefix: next token, then per depth k a chain draft and its runner-up
    (both children of the previous chain node)."""
    nodes = [(int(ids[0]), 0, P, 1)]
    for k in range(8):
        par = 0 if k == 0 else 2 * k - 1
        nodes.append((int(ids[1 + 2 * k]), 0, P + 1 + k, 1, P + 1 + 2 * k, par))
        nodes.append((int(ids[2 + 2 * k]), 0, P + 1 + k, 1, P + 2 + 2 * k, par))
    return nodes


def rows_probe():
    """Launch sequence for the prefill attention's counters (rocprofv3 --pmc): k_attention_rows on the pp512 forward's
    shape (512 causal tokens of one sequence, 32 query heads over 8 KV heads, head_dim 128, keys 1..512 per token) over
    a random int8 KV cache, 3 untimed launches then 20."""
    import ctypes
    import malkin_amd as mk
    L = mk.load()
    ctx = mk.Context(0)
    rng = np.random.default_rng(7)
    D, H, KV, n_ctx, n = 128, 32, 8, 4096, N_PROMPT
    k8 = ctx.to_device(rng.integers(-127, 128, (1, KV, n_ctx, D), dtype=np.int8))
    v8 = ctx.to_device(rng.integers(-127, 128, (1, KV, n_ctx, D), dtype=np.int8))
    ks = ctx.to_device(rng.uniform(0.001, 0.05, (1, KV, n_ctx)).astype(np.float32))
    vs = ctx.to_device(rng.uniform(0.001, 0.05, (1, KV, n_ctx)).astype(np.float32))
    kv = mk.MkKvCache(k8.ptr, v8.ptr, ks.ptr, vs.ptr, 1, 1, KV, D, n_ctx)
    q = ctx.to_device(rng.standard_normal((n, H * D)).astype(np.float32))
    seq = ctx.to_device(np.zeros(n, np.int32))
    nk = ctx.to_device(np.arange(1, n + 1, dtype=np.int32))
    out = ctx.alloc(n * H * D * 4)
    for i in range(23):
        mk.check(L.mk_attention(ctx.h, q.ptr, H * D, out.ptr, H * D, n, H, ctypes.byref(kv), 0, seq.ptr, nk.ptr, None,
                                None, n))
    ctx.sync()
    log(f"[probe] k_attention_rows: {n} causal tokens, {H} heads over {KV} KV heads, head_dim {D}: 23 launches")
    ctx.close()


def tree_probe():
    """Launch sequence for the tree-verification kernel trace: config 5's target (Qwen3-14B shape, Q6_K), the
    2048-token prefix in 256-token forwards, then 4 verifications of the 17-node tree."""
    import malkin_amd as mk
    from malkin_amd import synth
    rng = np.random.default_rng(5)
    tpath, _ = model_file("qwen3-14b", seed=5, wtype=synth.Q6_K)
    try:
        ctx = mk.Context(0)
        t = mk.Model(ctx, tpath, N_CTX, 1)
        P = 2048
        prompt = rng.integers(0, t.cfg["n_vocab"], size=P).astype(np.int32)
        for i in range(0, P, 256):
            t.forward(prompt[i:i + 256], i)
        tree = mk.batch(tree_nodes(rng.integers(0, t.cfg["n_vocab"], size=17), P))
        for i in range(4):
            t.forward_top2(tree)
            ctx.sync()
            log(f"[probe] verification {i}")
        t.close()
        ctx.close()
    finally:
        if os.path.exists(tpath):
            os.remove(tpath)


def config5(ctx):
    """target Qwen3-14B in Q6_K, draft Qwen3-0.6B in Q4_K_M, 2048-token prefix. (a) One tree
    verification: the target forward of 17 nodes (next token + a chain of 8 drafts + one runner-up per depth, the
    engine's tree layout) with the tree attention mask over the 2048-token KV prefix, greedy picks on the device; (b)
    the speculative engine (draft chain / runner-up tree, n_draft 8) generating 64 tokens after that prompt."""
    import malkin_amd as mk
    from malkin_amd import synth
    rng = np.random.default_rng(5)
    tpath, _ = model_file("qwen3-14b", seed=5, wtype=synth.Q6_K)
    dpath, _ = model_file("qwen3-0.6b", seed=6, wtype=synth.Q4_K, mix=synth.MIX_Q4_K_M)
    try:
        t = mk.Model(ctx, tpath, N_CTX, 1)
        d = mk.Model(ctx, dpath, N_CTX, 1)
        V = t.cfg["n_vocab"]
        P = 2048
        prompt = rng.integers(0, V, size=P).astype(np.int32)
        ctx.sync()
        t0 = time.perf_counter()
        for i in range(0, P, 256):
            t.forward(prompt[i:i + 256], i)
        ctx.sync()
        prefill_s = time.perf_counter() - t0
        tree = mk.batch(tree_nodes(rng.integers(0, V, size=17), P))
        t.forward_top2(tree)
        ctx.sync()
        reps = 10
        t0 = time.perf_counter()
        for _ in range(reps):
            t.forward_top2(tree)
        ctx.sync()
        verify_ms = (time.perf_counter() - t0) * 1e3 / reps
        e = mk.Engine(t, d, 8)
        ctx.sync()
        t0 = time.perf_counter()
        rid = e.submit(prompt, 64)
        e.run()
        ctx.sync()
        wall = time.perf_counter() - t0
        _, info = e.result(rid)
        e.close()
        d.close()
        t.close()
    finally:
        for p in (tpath, dpath):
            if os.path.exists(p):
                os.remove(p)
    return {"workload": "qwen3-14b-q6_k target + qwen3-0.6b-q4_k_m draft, 2048-token prompt (random ids), tree of "
                        "17 nodes per verification",
            "verify_ms": round(verify_ms, 3), "verify_nodes": 17, "prefix_prefill_tok_s": round(P / prefill_s, 1),
            "spec_gen_tokens": info["completion_tokens"], "spec_wall_s": round(wall, 3),
            "spec_decode_tok_s": round(info["completion_tokens"] * 1e3 / max(info["decode_ms"], 1e-9), 1),
            "drafted": info["drafted"], "accepted": info["accepted"],
            "note": "random-init target and draft agree on almost no token, so nearly every verification accepts "
                    "only its root; verify_ms is the per-pass cost"}


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
    ap.add_argument("--no-kernel-configs", action="store_true",
                    help="skip the kernel-level configurations (config 1 GEMM, config 2 GEMV)")
    ap.add_argument("--no-engine-configs", action="store_true",
                    help="skip BASELINE configs 3 (Qwen3-4B pp512 + tg128), 4 (continuous batching) and 5 "
                         "(speculative tree verification)")
    ap.add_argument("--probe", choices=["traffic", "decode", "gemm", "kquant", "tree", "rows"],
                    help="only run a launch sequence for counter profiles: the roofline kernel's HBM traffic, "
                         "one decode layer's kernels (attention and the four GEMVs, for instruction and wait counters), "
                         "the prefill GEMM (config 1 and the pp512 forward's shapes), config 2's short K-quant batches, "
                         "config 5's tree verification, or the pp512 forward's prefill attention")
    args = ap.parse_args()
    if args.probe == "traffic":
        traffic_probe()
        return
    if args.probe == "decode":
        decode_probe()
        return
    if args.probe == "gemm":
        gemm_probe()
        return
    if args.probe == "kquant":
        kquant_probe()
        return
    if args.probe == "tree":
        tree_probe()
        return
    if args.probe == "rows":
        rows_probe()
        return
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
        # The reference engine's prefill protocol (two 256-token forwards, engine.cpp:381-393), outside the timed step.
        pp2 = []
        for i in range(3):
            ctx.sync()
            t1 = time.perf_counter()
            for c in range(0, N_PROMPT, 256):
                model.forward(prompt[c:c + 256], c)
            ctx.sync()
            pp2.append(time.perf_counter() - t1)
        log(f"[bench] pp512 in two 256-token forwards: {min(pp2) * 1e3:.2f} ms (best of 3)")
        roof = gemv_roofline(ctx, model, cfg)
        log(f"[bench] decode GEMV: {roof['achieved']} GB/s ({roof['us_per_launch']} us per launch)")
        model.close()
        kern = None if args.no_kernel_configs else kernel_configs(ctx)
        if kern:
            log("[bench] kernel configs: " + json.dumps(kern))
        engine = None
        if not args.no_engine_configs:
            engine = {"config3": config3(ctx, with_cpu=not args.no_cpu_baseline, use_graph=not args.no_graph)}
            log("[bench] config 3: " + json.dumps(engine["config3"]))
            engine["config4"] = config4(ctx, path)
            log("[bench] config 4: " + json.dumps(engine["config4"]))
            engine["config5"] = config5(ctx)
            log("[bench] config 5: " + json.dumps(engine["config5"]))
        cpu = None if args.no_cpu_baseline else cpu_baseline(path, prompt, toks)
        if cpu:
            log("[bench] cpu baseline: " + json.dumps(cpu))
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
        "pp512_2x256_tok_s": round(N_PROMPT / float(np.median(pp2)), 1),
        "tg128_tok_s": round((N_GEN - 1) * 1e3 / dec_ms, 2),
        "decode_ms_per_token": round(dec_ms / (N_GEN - 1), 4),
        "decode_hbm_frac": round(model_bytes_per_token(cfg) / (dec_ms / (N_GEN - 1) / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
        "pp512_mfma_frac": round(prefill_ops(cfg) / (pp_ms / 1e3) / 1e12 / INT8_PEAK_TOPS, 4),
        "tokens_match": None if cpu is None else cpu.get("tokens_match"),
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernel_configs": kern,
        "engine_configs": engine,
    }
    print(json.dumps(line), flush=True)


def prefill_ops(cfg):
    """Algorithmic int8 ops of the pp512 prefill: 2 * 512 * (weights of the layer matmuls); the LM head runs on the
    last token only."""
    E, F, H, KV, D, L = (cfg[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_layer"))
    return 2.0 * N_PROMPT * L * ((H + 2 * KV) * D * E + E * H * D + 3 * F * E)


def model_bytes_per_token(cfg):
    """Algorithmic bytes of one decode token: GGUF bytes of every matmul weight read (incl. the LM head)."""
    E, F, H, KV, D, V, L = (cfg[k] for k in ("n_embd", "n_ff", "n_head", "n_head_kv", "head_dim", "n_vocab",
                                              "n_layer"))
    per_layer = ((H + 2 * KV) * D * E + E * H * D + 2 * F * E + E * F) // 32 * 34
    return per_layer * L + V * E // 32 * 34


if __name__ == "__main__":
    main()
