"""malkin-mi355x: Python bindings (ctypes) over the C ABI of libmalkin_hip.so.

The C ABI (include/malkin_hip.h, include/malkin_model.h) is the product; this module only loads it for the tests and
the benchmark. There is no fallback: if the library is missing, load() raises.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmalkin_hip.so")

MK_OK, MK_ERR_INVALID, MK_ERR_HIP, MK_ERR_UNSUPPORTED, MK_ERR_NO_DEVICE = 0, 1, 2, 3, 4
F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 8, 12, 13, 14, 30
MODEL_NO_WIDE, MODEL_NO_PACK, MODEL_PERSISTENT, MODEL_FUSED_ATTN = 1, 2, 4, 8

BLOCK_Q8 = np.dtype([("d", "<f4"), ("s", "<i2", (2,)), ("qs", "i1", (32,))])
BATCH_TOKEN = np.dtype([("id", "<i4"), ("seq", "<i4"), ("pos", "<i4"), ("logits", "<i4"), ("kv", "<i4"),
                        ("parent", "<i4")])

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_SZ = ctypes.c_size_t
_F = ctypes.c_float

# name -> (restype, argtypes); the exports of include/malkin_hip.h and include/malkin_model.h
SIGNATURES = {
    "mk_init": (_I, [_I, ctypes.POINTER(_P)]),
    "mk_destroy": (_I, [_P]),
    "mk_device_name": (ctypes.c_char_p, [_P]),
    "mk_last_error": (ctypes.c_char_p, []),
    "mk_synchronize": (_I, [_P]),
    "mk_reserve_scratch": (_I, [_P, _SZ]),
    "mk_attention_scratch_bytes": (_SZ, [_I, _I, _I]),
    "mk_stream": (_P, [_P]),
    "mk_malloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "mk_free": (_I, [_P, _P]),
    "mk_upload": (_I, [_P, _P, _P, _SZ]),
    "mk_download": (_I, [_P, _P, _P, _SZ]),
    "mk_fill": (_I, [_P, _P, _I, _SZ]),
    "mk_timer_start": (_I, [_P]),
    "mk_timer_stop": (_I, [_P, ctypes.POINTER(_F)]),
    "mk_packed_bytes": (_SZ, [_I, _I64, _I64]),
    "mk_pack_weight": (_I, [_P, _I, _P, _SZ, _I64, _I64, _P]),
    "mk_pack_weight_rows": (_I, [_P, _I, _P, _SZ, _I64, _I64, _I64, _I64, _P]),
    "mk_unpack_weight": (_I, [_P, _I, _P, _I64, _I64, _P]),
    "mk_quantize_q8": (_I, [_P, _P, _I, _I64, _P]),
    "mk_quantize_i8": (_I, [_P, _P, _I, _I, _P, _P]),
    "mk_dequantize_rows": (_I, [_P, _I, _P, _SZ, _P, _I, _I64, _P]),
    "mk_matmul": (_I, [_P, _P, _P, _I, _P, _I64, _I]),
    "mk_matmul_f32": (_I, [_P, _P, _P, _I64, _P, _F, _I, _P, _I64, _I, _I]),
    "mk_rmsnorm": (_I, [_P, _P, _P, _I, _I, _F, _P]),
    "mk_rmsnorm_q8": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "mk_silu_mul": (_I, [_P, _I64, _P, _P]),
    "mk_rmsnorm_rows": (_I, [_P, _P, _P, _P, _I, _I, _F, _P]),
    "mk_silu_mul_rows": (_I, [_P, _P, _I, _I64]),
    "mk_matmul_gguf": (_I, [_P, _I, _P, _SZ, _I64, _I64, _P, _I, _P, _I64, _I]),
    "mk_matmul_rows": (_I, [_P, _I, _P, _SZ, _I64, _I64, _P, _I64, _P, _I, _P, _I64, _I]),
    "mk_silu_mul_q8": (_I, [_P, _P, _I, _I64, _I, _P]),
    "mk_add": (_I, [_P, _I64, _P, _P]),
    "mk_attend_gqa": (_I, [_P, _P, _I, _I, _P, _P, _SZ, ctypes.c_ssize_t, _I, _F, _P, _P, _I]),
    "mk_qk_norm_rope_kv": (_I, [_P, _P, _P, _P, _I64, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P, _I]),
    "mk_attention": (_I, [_P, _P, _I64, _P, _I64, _I, _I, _P, _I, _P, _P, _P, _P, _I]),
    "mk_attention_decode": (_I, [_P, _P, _I64, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _I]),
    "mk_attention_q8": (_I, [_P, _P, _I64, _P, _I64, _I, _I, _P, _I, _P, _P, _P, _P, _I, _P]),
    "mk_attention_decode_q8": (_I, [_P, _P, _I64, _I, _I, _P, _P, _F, _P, _P, _P, _P, _P, _P, _P, _I, _P, _I64, _I,
                                    _P]),
    "mk_move_kv": (_I, [_P, _P, _I, _I, _I]),
    "mk_decode_plan_create": (_I, [_P, _P, _I, _I, _F, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, ctypes.POINTER(_P)]),
    "mk_decode_plan_destroy": (_I, [_P]),
    "mk_decode_supported": (_I, [_P, _I]),
    "mk_decode_layers": (_I, [_P, _P, _I, _I, _I]),
    "mk_decode_check": (_I, [_P, _P]),
    "mk_decode_attn_wo": (_I, [_P, _P, _I, _I]),
    "mk_model_persistent": (_I, [_P]),
    "mk_model_eog": (_I, [_P, _P, _I]),
    "mk_argmax_top2": (_I, [_P, _P, _I, _I, _P, _P]),
    "mk_greedy_advance": (_I, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "mk_argmax_top2_noalloc": (_I, [_P, _P, _I, _I, _P, _P]),
    "mk_host_waits": (ctypes.c_uint64, []),
    "mk_host_bytes": (ctypes.c_uint64, []),
    "mk_host_alloc": (_I, [_P, _SZ, ctypes.POINTER(_P)]),
    "mk_host_free": (_I, [_P, _P]),
    "mk_copy_async": (_I, [_P, _P, _P, _SZ]),
    "mk_event_record": (_I, [_P, ctypes.POINTER(_P)]),
    "mk_event_wait": (_I, [_P, _P]),
    "mk_event_done": (_I, [_P]),
    "mk_event_free": (_I, [_P]),
    "mk_move_ids": (_I, [_P, _P, _P, _P, _P, _I]),
    "mk_gguf_inspect": (_I, [ctypes.c_char_p, _P]),
    "mk_model_open": (_I, [_P, ctypes.c_char_p, _I, _I, _I, ctypes.POINTER(_P)]),
    "mk_model_free": (_I, [_P]),
    "mk_model_get_config": (_I, [_P, _P]),
    "mk_model_forward_batch": (_I, [_P, _P, _I, _P]),
    "mk_model_forward": (_I, [_P, _P, _I, _I, _P, _I, _P, _I]),
    "mk_model_forward_top2": (_I, [_P, _P, _I, _P, _P]),
    "mk_model_move_kv": (_I, [_P, _I, _I, _I]),
    "mk_model_kv_row": (_I, [_P, _I, _I, _I, _I, _P]),
    "mk_model_generate": (_I, [_P, _P, _I, _I, _I, _I, _P, _P]),
    "mk_model_weight_bytes": (_I64, [_P]),
    "mk_model_weight": (_I, [_P, _I, _I, _P]),
    "mk_engine_create": (_I, [_P, _P, _I, ctypes.POINTER(_P)]),
    "mk_engine_free": (_I, [_P]),
    "mk_engine_submit": (_I, [_P, _P, _I, _I, _P, _I, _P]),
    "mk_engine_step": (_I, [_P, _P]),
    "mk_engine_run": (_I, [_P]),
    "mk_engine_steps": (_I, [_P, ctypes.POINTER(ctypes.c_uint64)]),
    "mk_engine_draws": (_I, [_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "mk_engine_result": (_I, [_P, _I, _P, _I, _P]),
    "mk_engine_release": (_I, [_P, _I, ctypes.POINTER(ctypes.c_int64)]),
    "mk_engine_submit_sampled": (_I, [_P, _P, _I, _I, _P, _I, _P, _P]),
    "mk_penalize": (_I, [_P, _P, _I64, _P, _I, _I, _P, _P, _P]),
    "mk_topk": (_I, [_P, _P, _I64, _P, _I, _I, _I, _P, _P]),
    "mk_sample_cut_workspace": (ctypes.c_size_t, [_I, _I]),
    "mk_sample_cut": (_I, [_P, _P, _I64, _P, _I, _I, _P, _I, _P, _P, _P, _P, _P, ctypes.c_size_t]),
    "mk_sample_cut_tail": (_I, [_P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "mk_sample_draw": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _P, _I]),
    "mk_server_start": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p, _I, ctypes.POINTER(_P), ctypes.POINTER(_I)]),
    "mk_server_stop": (_I, [_P]),
    "mk_sampler_create": (_I, [_P, _I, ctypes.POINTER(_P)]),
    "mk_sampler_free": (_I, [_P]),
    "mk_sampler_accept": (_I, [_P, ctypes.c_int32]),
    "mk_sampler_distribution": (_I, [_P, _P, _P, _I, _P, _P, _I, ctypes.POINTER(_I)]),
    "mk_sampler_sample": (_I, [_P, _P, _P, _I, ctypes.POINTER(ctypes.c_int32)]),
    "mk_sampler_draw": (_I, [_P, _P, _P, _I, ctypes.POINTER(ctypes.c_int32)]),
    "mk_sampler_verify": (_I, [_P, _P, _P, _I, _P, _P, _I, ctypes.c_int32, ctypes.POINTER(_I),
                               ctypes.POINTER(ctypes.c_int32)]),
}

_lib = None


class MkError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


def load():
    """The native library; raises if it is not built (there is no non-native path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def check(rc):
    if rc != MK_OK:
        raise MkError(rc, load().mk_last_error().decode())


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


class Buffer:
    """Device allocation (mk_malloc) with numpy upload/download helpers."""

    def __init__(self, ctx, nbytes):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p = _P()
        check(load().mk_malloc(ctx.h, max(1, self.nbytes), ctypes.byref(p)))
        self.p = p.value

    @property
    def ptr(self):
        return ctypes.c_void_p(self.p)

    def offset(self, nbytes):
        return ctypes.c_void_p(self.p + int(nbytes))

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(load().mk_upload(self.ctx.h, self.offset(offset), _ptr(arr), arr.nbytes))
        return self

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        check(load().mk_download(self.ctx.h, _ptr(out), self.offset(offset), out.nbytes))
        return out

    def free(self):
        # After the context is destroyed its allocations are gone with it; nothing left to free.
        if self.p and self.ctx.h:
            load().mk_free(self.ctx.h, ctypes.c_void_p(self.p))
        self.p = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    def __init__(self, device=0):
        p = _P()
        check(load().mk_init(device, ctypes.byref(p)))
        self.h = p.value

    def close(self):
        if self.h:
            load().mk_destroy(self.h)
            self.h = None

    @property
    def device_name(self):
        return load().mk_device_name(self.h).decode()

    def sync(self):
        check(load().mk_synchronize(self.h))

    def alloc(self, nbytes):
        return Buffer(self, nbytes)

    def to_device(self, arr):
        arr = np.ascontiguousarray(arr)
        return Buffer(self, arr.nbytes).upload(arr)

    def timer_start(self):
        check(load().mk_timer_start(self.h))

    def timer_stop(self):
        ms = _F()
        check(load().mk_timer_stop(self.h, ctypes.byref(ms)))
        return ms.value


class MkWeight(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("wide", ctypes.c_int32), ("rows", ctypes.c_int64),
                ("cols", ctypes.c_int64), ("data", ctypes.c_void_p)]


class MkDecodeLayer(ctypes.Structure):
    _fields_ = [("qkv", MkWeight), ("wo", MkWeight), ("gate_up", MkWeight), ("down", MkWeight),
                ("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p), ("q_norm", ctypes.c_void_p),
                ("k_norm", ctypes.c_void_p)]


class MkKvCache(ctypes.Structure):
    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("k_scale", ctypes.c_void_p),
                ("v_scale", ctypes.c_void_p), ("n_layer", ctypes.c_int32), ("n_seq", ctypes.c_int32),
                ("n_head_kv", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("n_ctx", ctypes.c_int32)]


class MkModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim",
                                              "n_vocab", "n_ctx", "n_seq")] + [("rope_base", ctypes.c_float),
                                                                              ("rms_eps", ctypes.c_float)]


class MkGenStats(ctypes.Structure):
    _fields_ = [("prefill_ms", ctypes.c_double), ("decode_ms", ctypes.c_double), ("decode_forwards", ctypes.c_int32)]


class MkGgufInfo(ctypes.Structure):
    _fields_ = [("n_tensors", ctypes.c_int64), ("tensor_bytes", ctypes.c_int64), ("n_layer", ctypes.c_int32),
                ("arch", ctypes.c_char * 32), ("n_eog", ctypes.c_int32), ("eog", ctypes.c_int32 * 8)]


def gguf_inspect(path):
    """mk_gguf_inspect: validates a GGUF file on the host (no device needed); raises MkError with the reason."""
    info = MkGgufInfo()
    check(load().mk_gguf_inspect(path.encode(), ctypes.byref(info)))
    out = {"n_tensors": info.n_tensors, "tensor_bytes": info.tensor_bytes, "n_layer": info.n_layer,
           "arch": info.arch.decode()}
    if info.n_eog:
        out["eog"] = list(info.eog[:min(info.n_eog, 8)])
    return out


class Model:
    """mk_model_* wrapper: the device counterpart of the reference's Model (model.h)."""

    def __init__(self, ctx, path, n_ctx, n_seq=1, wide=True, no_pack=False, persistent=False, fused_attn=False):
        self.ctx = ctx
        p = _P()
        flags = ((0 if wide else MODEL_NO_WIDE) | (MODEL_NO_PACK if no_pack else 0) |
                 (MODEL_PERSISTENT if persistent else 0) | (MODEL_FUSED_ATTN if fused_attn else 0))
        check(load().mk_model_open(ctx.h, path.encode(), n_ctx, n_seq, flags, ctypes.byref(p)))
        self.h = p.value
        c = MkModelConfig()
        check(load().mk_model_get_config(self.h, ctypes.byref(c)))
        self.cfg = {f: getattr(c, f) for f, _ in MkModelConfig._fields_}

    def close(self):
        if self.h and self.ctx.h:
            load().mk_model_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def persistent(self):
        """One-token forwards in the persistent decode kernel (every layer in one launch)."""
        return load().mk_model_persistent(self.h) == 1

    @property
    def fused_attn(self):
        """One-token forwards with each layer's attention and attn_output in one launch."""
        return load().mk_model_persistent(self.h) == 2

    @property
    def eog(self):
        """The model's end-of-generation ids (the GGUF's eos / eot / eom ids and end-of-turn control tokens)."""
        n = load().mk_model_eog(self.h, None, 0)
        if n < 0:
            check(n)
        out = np.zeros(max(n, 1), np.int32)
        check(min(0, load().mk_model_eog(self.h, out.ctypes.data, n)))
        return [int(v) for v in out[:n]]

    @property
    def weight_bytes(self):
        return int(load().mk_model_weight_bytes(self.h))

    def weight(self, layer, which):
        w = MkWeight()
        check(load().mk_model_weight(self.h, layer, which, ctypes.byref(w)))
        return w

    def forward_batch(self, batch):
        batch = np.ascontiguousarray(batch, dtype=BATCH_TOKEN)
        nl = int((batch["logits"] != 0).sum())
        logits = np.zeros((max(nl, 1), self.cfg["n_vocab"]), dtype=np.float32)
        check(load().mk_model_forward_batch(self.h, _ptr(batch), len(batch), _ptr(logits)))
        return logits[:nl]

    def forward(self, tokens, pos, all_logits=False, parent=None, seq=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        logits = np.zeros((n if all_logits else 1, self.cfg["n_vocab"]), dtype=np.float32)
        par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
        check(load().mk_model_forward(self.h, _ptr(tokens), n, pos, _ptr(logits), 1 if all_logits else 0, _ptr(par),
                                      seq))
        return logits

    def forward_top2(self, batch):
        batch = np.ascontiguousarray(batch, dtype=BATCH_TOKEN)
        nl = int((batch["logits"] != 0).sum())
        t1 = np.zeros(max(nl, 1), dtype=np.int32)
        t2 = np.zeros(max(nl, 1), dtype=np.int32)
        check(load().mk_model_forward_top2(self.h, _ptr(batch), len(batch), _ptr(t1), _ptr(t2)))
        return t1[:nl], t2[:nl]

    def move_kv(self, frm, to, seq=0):
        check(load().mk_model_move_kv(self.h, frm, to, seq))

    def kv_row(self, layer, seq, pos, k=True):
        nb = self.cfg["n_head_kv"] * (self.cfg["head_dim"] + 4)
        out = np.zeros(nb, dtype=np.int8)
        check(load().mk_model_kv_row(self.h, layer, seq, pos, 1 if k else 0, _ptr(out)))
        return out

    def generate(self, prompt, n_gen, seq=0, use_graph=True):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_gen, dtype=np.int32)
        st = MkGenStats()
        check(load().mk_model_generate(self.h, _ptr(prompt), len(prompt), n_gen, seq, 1 if use_graph else 0,
                                       _ptr(out), ctypes.byref(st)))
        return out, {"prefill_ms": st.prefill_ms, "decode_ms": st.decode_ms, "decode_forwards": st.decode_forwards}


class MkRequestInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("prompt_tokens", "cached_tokens", "completion_tokens", "drafted",
                                              "accepted", "finish", "done")] + [("prefill_ms", ctypes.c_double),
                                                                                 ("decode_ms", ctypes.c_double)]


class Engine:
    """mk_engine_* wrapper: continuous batching and greedy speculative decoding over Model (engine.h)."""

    def __init__(self, target, draft=None, n_draft=0):
        self.target, self.draft = target, draft  # keep the models alive
        p = _P()
        check(load().mk_engine_create(target.h, draft.h if draft is not None else None, n_draft, ctypes.byref(p)))
        self.h = p.value

    def close(self):
        if self.h:
            load().mk_engine_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def submit(self, prompt, max_tokens=0, eog=(), sampling=None):
        """sampling: None (greedy) or SamplingParams fields as keywords of sampling_params()."""
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        eog = np.ascontiguousarray(list(eog), dtype=np.int32)
        rid = ctypes.c_int32()
        if sampling is None:
            check(load().mk_engine_submit(self.h, _ptr(prompt), len(prompt), max_tokens,
                                          _ptr(eog) if len(eog) else None, len(eog), ctypes.byref(rid)))
        else:
            sp = sampling_params(**sampling)
            check(load().mk_engine_submit_sampled(self.h, _ptr(prompt), len(prompt), max_tokens,
                                                  _ptr(eog) if len(eog) else None, len(eog), ctypes.byref(sp),
                                                  ctypes.byref(rid)))
        return rid.value

    def step(self):
        busy = ctypes.c_int32()
        check(load().mk_engine_step(self.h, ctypes.byref(busy)))
        return busy.value

    def run(self):
        check(load().mk_engine_run(self.h))

    @property
    def steps(self):
        n = ctypes.c_uint64()
        check(load().mk_engine_steps(self.h, ctypes.byref(n)))
        return n.value

    @property
    def draws(self):
        """(drafts drawn on the device, of which the host's replay drew differently)."""
        a, b = ctypes.c_uint64(), ctypes.c_uint64()
        check(load().mk_engine_draws(self.h, ctypes.byref(a), ctypes.byref(b)))
        return a.value, b.value

    def result(self, rid):
        info = MkRequestInfo()
        check(load().mk_engine_result(self.h, rid, None, 0, ctypes.byref(info)))
        toks = np.zeros(max(info.completion_tokens, 1), dtype=np.int32)
        check(load().mk_engine_result(self.h, rid, _ptr(toks), len(toks), ctypes.byref(info)))
        return toks[:info.completion_tokens], {f: getattr(info, f) for f, _ in MkRequestInfo._fields_}

    def release(self, rid):
        """Frees a finished request's result; returns the number of results still held."""
        held = ctypes.c_int64()
        check(load().mk_engine_release(self.h, rid, ctypes.byref(held)))
        return held.value


class Server:
    """mk_server_*: the HTTP API (include/malkin_server.h) over an Engine (None: health and models only), on
    host:port (0: a free port, then .port)."""

    def __init__(self, engine=None, model_id="malkin", host="127.0.0.1", port=0):
        self.engine = engine
        p, bound = _P(), _I()
        check(load().mk_server_start(engine.h if engine is not None else None, model_id.encode(), host.encode(), port,
                                     ctypes.byref(p), ctypes.byref(bound)))
        self.h, self.port = p.value, bound.value

    def close(self):
        if self.h:
            load().mk_server_stop(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MkSamplingParams(ctypes.Structure):
    _fields_ = [("temperature", _F), ("top_p", _F), ("top_k", ctypes.c_int32), ("min_p", _F),
                ("presence_penalty", _F), ("frequency_penalty", _F), ("seed", ctypes.c_uint64)]


def sampling_params(temperature=0.8, top_p=0.95, top_k=40, min_p=0.05, presence=0.0, frequency=0.0, seed=0):
    """mk_sampling_params with the reference's defaults (sampler.h:10-18)."""
    return MkSamplingParams(temperature, top_p, top_k, min_p, presence, frequency, seed)


class Sampler:
    """mk_sampler_*: the reference's Sampler (sampler.h:23-42) with its distribution over device logits rows.
    Distributions are [(p, id), ...] lists, highest first."""

    def __init__(self, seed, penalties=True, **params):
        sp = sampling_params(seed=seed, **params)
        p = _P()
        check(load().mk_sampler_create(ctypes.byref(sp), 1 if penalties else 0, ctypes.byref(p)))
        self.h = p.value

    def close(self):
        if self.h:
            load().mk_sampler_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def accept(self, tok):
        check(load().mk_sampler_accept(self.h, int(tok)))

    def distribution(self, ctx, dev_logits, n_vocab):
        """dev_logits: DeviceBuffer (or device pointer) of one row; penalized in place."""
        ptr = dev_logits.ptr if hasattr(dev_logits, "ptr") else dev_logits
        cap = n_vocab
        probs = np.zeros(cap, np.float32)
        ids = np.zeros(cap, np.int32)
        n = ctypes.c_int()
        check(load().mk_sampler_distribution(ctx.h, self.h, ptr, n_vocab, _ptr(probs), _ptr(ids), cap,
                                             ctypes.byref(n)))
        return [(float(probs[i]), int(ids[i])) for i in range(n.value)]

    def sample(self, ctx, dev_logits, n_vocab):
        ptr = dev_logits.ptr if hasattr(dev_logits, "ptr") else dev_logits
        t = ctypes.c_int32()
        check(load().mk_sampler_sample(ctx.h, self.h, ptr, n_vocab, ctypes.byref(t)))
        return t.value

    def draw(self, d):
        pp = np.ascontiguousarray([e[0] for e in d], np.float32)
        pi = np.ascontiguousarray([e[1] for e in d], np.int32)
        t = ctypes.c_int32()
        check(load().mk_sampler_draw(self.h, _ptr(pp), _ptr(pi), len(pp), ctypes.byref(t)))
        return t.value

    def verify(self, p, q, draft):
        pp = np.ascontiguousarray([e[0] for e in p], np.float32)
        pi = np.ascontiguousarray([e[1] for e in p], np.int32)
        qp = np.ascontiguousarray([e[0] for e in q] or [0.0], np.float32)
        qi = np.ascontiguousarray([e[1] for e in q] or [0], np.int32)
        a, t = ctypes.c_int(), ctypes.c_int32()
        check(load().mk_sampler_verify(self.h, _ptr(pp), _ptr(pi), len(pp), _ptr(qp), _ptr(qi), len(q), int(draft),
                                       ctypes.byref(a), ctypes.byref(t)))
        return t.value, bool(a.value)


def host_waits():
    """Host waits on the device the library has made so far (mk_host_waits)."""
    return int(load().mk_host_waits())


def batch(tokens):
    """Structured BatchToken array from (id, seq, pos, logits[, kv, parent]) tuples."""
    out = np.zeros(len(tokens), dtype=BATCH_TOKEN)
    for i, t in enumerate(tokens):
        t = tuple(t) + (-1, -1)[len(t) - 4:] if len(t) < 6 else tuple(t)
        out[i] = t[:6]
    return out
