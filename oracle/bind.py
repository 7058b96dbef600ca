"""ctypes bindings of the CPU oracle (liboracle.so, the C restatement) and of the compiled reference
(_ref/libmalkin_ref.so). TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker; the product path never imports it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libmalkin_ref.so")

F32, F16, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 8, 12, 13, 14, 30

# BlockQ8 (quant.h:11-16): float d; int16 s[2]; int8 qs[32] -> 40 bytes.
BLOCK_Q8 = np.dtype([("d", "<f4"), ("s", "<i2", (2,)), ("qs", "i1", (32,))])
assert BLOCK_Q8.itemsize == 40

BATCH_TOKEN = np.dtype([("id", "<i4"), ("seq", "<i4"), ("pos", "<i4"), ("logits", "<i4"), ("kv", "<i4"),
                        ("parent", "<i4")])

_P = ctypes.c_void_p


def ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


def row_size(t, k):
    return {F32: 4 * k, F16: 2 * k, BF16: 2 * k, Q8_0: k // 32 * 34, Q4_K: k // 256 * 144, Q5_K: k // 256 * 176,
            Q6_K: k // 256 * 210}[t]


class _Common:
    prefix = ""

    def _f(self, name):
        return getattr(self.lib, self.prefix + name)

    def quantize_row_q8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        k = x.shape[-1]
        out = np.zeros(x.size // 32, dtype=BLOCK_Q8)
        rows = x.reshape(-1, k)
        for i, r in enumerate(rows):
            self._f("quantize_row_q8")(ptr(r), ptr(out[i * (k // 32):]), ctypes.c_int64(k))
        return out.reshape(x.shape[:-1] + (k // 32,))

    def quantize_i8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.zeros(x.shape, dtype=np.int8)
        d = self._f("quantize_i8")(ptr(x), ctypes.c_int(x.size), ptr(q))
        return q, np.float32(d)

    def dequantize_row(self, t, data, k):
        out = np.zeros(k, dtype=np.float32)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        rc = self._f("dequantize_row")(ctypes.c_int(t), ptr(data), ptr(out), ctypes.c_int64(k))
        if rc != 0:
            raise RuntimeError("unsupported type")
        return out

    def dot_f32(self, w, x):
        w = np.ascontiguousarray(w, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        return np.float32(self._f("dot_f32")(ctypes.c_int64(w.size), ptr(w), ptr(x)))

    def silu_mul(self, g, u):
        g = np.array(g, dtype=np.float32, copy=True)
        u = np.ascontiguousarray(u, dtype=np.float32)
        self._f("silu_mul")(ctypes.c_int64(g.size), ptr(g), ptr(u))
        return g

    def vec_dot(self, t, k, w, x=None, xq=None):
        """vec_dot (quant.cpp:171-191): one weight row (GGUF bytes) . one activation row (fp32 x or BlockQ8 xq)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = None if x is None else np.ascontiguousarray(x, dtype=np.float32)
        xq = None if xq is None else np.ascontiguousarray(xq, dtype=BLOCK_Q8)
        f = self._f("vec_dot")
        f.restype = ctypes.c_float
        return np.float32(f(ctypes.c_int(t), ctypes.c_int64(k), ptr(w), ptr(x), ptr(xq)))

    def attend_gqa(self, q, G, D, k, v, stride, soff, n, scale, extra=None):
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.zeros(G * D, dtype=np.float32)
        ne = 0 if extra is None else len(extra)
        scratch = np.zeros(G * (n + ne) + 16, dtype=np.float32)
        ex = None if extra is None else np.ascontiguousarray(extra, dtype=np.int32)
        self._f("attend_gqa")(ptr(q), ctypes.c_int(G), ctypes.c_int(D), ptr(k), ptr(v), ctypes.c_size_t(stride),
                              ctypes.c_ssize_t(soff), ctypes.c_int(n), ctypes.c_float(scale), ptr(out), ptr(scratch),
                              ptr(ex), ctypes.c_int(ne))
        return out


class Oracle(_Common):
    """The C restatement (oracle.c)."""
    prefix = "or_"

    def __init__(self):
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} not built (make -C oracle)")
        L = self.lib = ctypes.CDLL(ORACLE_PATH)
        L.or_quantize_i8.restype = ctypes.c_float
        L.or_dot_f32.restype = ctypes.c_float
        L.or_exp.restype = ctypes.c_float
        L.or_exp.argtypes = [ctypes.c_float]
        L.or_reduce16.restype = ctypes.c_float
        L.or_fp16_to_fp32.restype = ctypes.c_float
        L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.or_fp32_to_fp16.restype = ctypes.c_uint16
        L.or_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.or_softmax_inplace.restype = ctypes.c_float
        L.or_argmax.restype = ctypes.c_int32
        L.or_model_open.restype = _P
        L.or_model_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                    ctypes.c_int]
        L.or_model_kv_row.restype = _P
        L.or_model_kv_row_bytes.restype = ctypes.c_size_t
        L.or_mt64_seed.argtypes = [_P, ctypes.c_uint64]
        L.or_mt64_next.restype = ctypes.c_uint64
        L.or_mt64_next.argtypes = [_P]
        L.or_mt64_uniform.restype = ctypes.c_double
        L.or_mt64_uniform.argtypes = [_P]
        L.or_penalize.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float, ctypes.c_float]
        L.or_distribution.argtypes = [_P, _P, ctypes.c_int, _P, _P]
        L.or_draw.restype = ctypes.c_int32
        L.or_draw.argtypes = [_P, _P, _P, ctypes.c_int]
        L.or_verify.restype = ctypes.c_int32
        L.or_verify.argtypes = [_P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int32, _P]
        L.or_verify_experiment.restype = ctypes.c_long
        L.or_verify_experiment.argtypes = [_P, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_uint64,
                                           ctypes.c_uint64, ctypes.c_long, _P, ctypes.c_int]

    def exp(self, x):
        return np.float32(self.lib.or_exp(ctypes.c_float(x)))

    def fp16_to_fp32(self, h):
        return np.float32(self.lib.or_fp16_to_fp32(int(h)))

    def fp32_to_fp16(self, f):
        return int(self.lib.or_fp32_to_fp16(ctypes.c_float(f)))

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        y = np.zeros_like(x)
        self.lib.or_rmsnorm(ptr(y), ptr(x), ptr(w), ctypes.c_int(x.size), ctypes.c_float(eps))
        return y

    def matmul(self, t, w, rows, cols, xq, wide=False):
        """y[t][r] for GGUF rows w (bytes), BlockQ8 activations xq [n][cols/32]."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=BLOCK_Q8)
        n = xq.size // (cols // 32)
        y = np.zeros((n, rows), dtype=np.float32)
        rc = self.lib.or_matmul(ctypes.c_int(t), ptr(w), ctypes.c_size_t(row_size(t, cols)), ctypes.c_int64(rows),
                                ctypes.c_int64(cols), ptr(xq), ctypes.c_int(n), ptr(y), ctypes.c_int64(rows),
                                ctypes.c_int(1 if wide else 0))
        if rc != 0:
            raise RuntimeError("or_matmul: unsupported type")
        return y

    def argmax(self, l):
        l = np.ascontiguousarray(l, dtype=np.float32)
        return int(self.lib.or_argmax(ptr(l), ctypes.c_int(l.size)))

    def top2(self, l):
        l = np.ascontiguousarray(l, dtype=np.float32)
        a, b = ctypes.c_int32(), ctypes.c_int32()
        self.lib.or_top2(ptr(l), ctypes.c_int(l.size), ctypes.byref(a), ctypes.byref(b))
        return a.value, b.value

    def matmul_rows(self, t, w, rows, cols, x=None, xq=None, n=1):
        """matmul's row path (quant.cpp:330-351)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = None if x is None else np.ascontiguousarray(x, dtype=np.float32)
        xq = None if xq is None else np.ascontiguousarray(xq, dtype=BLOCK_Q8)
        y = np.zeros((n, rows), dtype=np.float32)
        rc = self.lib.or_matmul_rows(ctypes.c_int(t), ptr(w), ctypes.c_size_t(row_size(t, cols)), ctypes.c_int64(rows),
                                     ctypes.c_int64(cols), ptr(x), ptr(xq), ctypes.c_int(n), ptr(y),
                                     ctypes.c_int64(rows))
        if rc != 0:
            raise RuntimeError("unsupported type")
        return y

    def model(self, path, n_ctx, n_seq=1, wide=True, no_pack=False):
        return OracleModel(self, path, n_ctx, n_seq, wide | (2 if no_pack else 0))

    def mt64(self, seed):
        return Mt64(self, seed)

    def sampler(self, seed, penalties=True, **params):
        return OracleSampler(self, seed, penalties, **params)

    def verify_experiment(self, p, q, target_seed, draft_seed, n_trials, V):
        """The reference's test_sampler.cpp experiment: (histogram of verified tokens, accepted count)."""
        pp, pi = _dist_arrays(p)
        qp, qi = _dist_arrays(q)
        hist = np.zeros(V, np.int64)
        acc = self.lib.or_verify_experiment(ptr(pp), ptr(pi), len(pp), ptr(qp), ptr(qi), len(qp), target_seed,
                                            draft_seed, n_trials, ptr(hist), V)
        return hist, int(acc)


SAMPLING_DEFAULTS = dict(temperature=0.8, top_p=0.95, top_k=40, min_p=0.05, presence=0.0, frequency=0.0)


def _dist_arrays(d):
    """[(p, id), ...] -> float32 probabilities, int32 ids."""
    return (np.ascontiguousarray([e[0] for e in d], np.float32), np.ascontiguousarray([e[1] for e in d], np.int32))


class _OrSampling(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_p", ctypes.c_float), ("top_k", ctypes.c_int),
                ("min_p", ctypes.c_float)]


class Mt64:
    """or_mt64: std::mt19937_64 and libstdc++'s uniform_real_distribution<double> on it."""

    def __init__(self, o, seed):
        self.o = o
        self.state = ctypes.create_string_buffer(312 * 8 + 8)
        o.lib.or_mt64_seed(self.state, seed)

    def next(self):
        return int(self.o.lib.or_mt64_next(self.state))

    def uniform(self):
        return float(self.o.lib.or_mt64_uniform(self.state))


class OracleSampler:
    """The reference's Sampler (sampler.h:23-42) over the oracle's C restatement: same methods, distributions as
    [(p, id), ...] lists, logits modified in place by the penalties."""

    def __init__(self, o, seed, penalties=True, **params):
        self.o, self.penalties = o, penalties
        self.p = dict(SAMPLING_DEFAULTS, **params)
        self.rng = Mt64(o, seed)
        self.counts = {}

    def accept(self, tok):
        self.counts[int(tok)] = self.counts.get(int(tok), 0) + 1

    def distribution(self, logits):
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        if self.penalties and self.counts:
            ids = np.array(list(self.counts.keys()), np.int32)
            cnt = np.array(list(self.counts.values()), np.int32)
            self.o.lib.or_penalize(ptr(logits), ptr(ids), ptr(cnt), len(ids), self.p["presence"], self.p["frequency"])
        sp = _OrSampling(self.p["temperature"], self.p["top_p"], self.p["top_k"], self.p["min_p"])
        probs = np.zeros(logits.size, np.float32)
        ids = np.zeros(logits.size, np.int32)
        n = self.o.lib.or_distribution(ctypes.byref(sp), ptr(logits), logits.size, ptr(probs), ptr(ids))
        return [(float(probs[i]), int(ids[i])) for i in range(n)]

    def draw(self, d):
        pp, pi = _dist_arrays(d)
        return int(self.o.lib.or_draw(self.rng.state, ptr(pp), ptr(pi), len(pp)))

    def sample(self, logits):
        return self.draw(self.distribution(logits))

    def verify(self, p, q, draft):
        pp, pi = _dist_arrays(p)
        qp, qi = _dist_arrays(q) if q else (np.zeros(1, np.float32), np.zeros(1, np.int32))
        a = ctypes.c_int()
        t = self.o.lib.or_verify(self.rng.state, ptr(pp), ptr(pi), len(pp), ptr(qp), ptr(qi), len(q), draft,
                                 ctypes.byref(a))
        return int(t), bool(a.value)


class _ModelBase:
    def config(self):
        return self.cfg

    def _err(self):
        return self.errbuf.value.decode()


class OracleModel(_ModelBase):
    def __init__(self, o, path, n_ctx, n_seq, wide):
        self.L = o.lib
        self.errbuf = ctypes.create_string_buffer(512)
        self.h = self.L.or_model_open(path.encode(), n_ctx, n_seq, int(wide), self.errbuf, 512)
        if not self.h:
            raise RuntimeError(self._err())
        c = (ctypes.c_int * 9)()
        self.L.or_model_config(_P(self.h), c)
        self.cfg = dict(n_layer=c[0], n_embd=c[1], n_ff=c[2], n_head=c[3], n_head_kv=c[4], head_dim=c[5],
                        n_vocab=c[6])
        self.n_ctx, self.n_seq = n_ctx, n_seq

    def close(self):
        if self.h:
            self.L.or_model_free(_P(self.h))
            self.h = None

    __del__ = close

    def forward_batch(self, batch):
        batch = np.ascontiguousarray(batch, dtype=BATCH_TOKEN)
        nl = int((batch["logits"] != 0).sum())
        logits = np.zeros((max(nl, 1), self.cfg["n_vocab"]), dtype=np.float32)
        rc = self.L.or_model_forward_batch(_P(self.h), ptr(batch), ctypes.c_int(len(batch)), ptr(logits), self.errbuf,
                                           512)
        if rc != 0:
            raise RuntimeError(self._err())
        return logits[:nl]

    def forward(self, tokens, pos, all_logits=False, parent=None, seq=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        logits = np.zeros((n if all_logits else 1, self.cfg["n_vocab"]), dtype=np.float32)
        par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
        rc = self.L.or_model_forward(_P(self.h), ptr(tokens), ctypes.c_int(n), ctypes.c_int(pos), ptr(logits),
                                     ctypes.c_int(1 if all_logits else 0), ptr(par), ctypes.c_int(seq), self.errbuf,
                                     512)
        if rc != 0:
            raise RuntimeError(self._err())
        return logits

    def move_kv(self, frm, to, seq=0):
        self.L.or_model_move_kv(_P(self.h), ctypes.c_int(frm), ctypes.c_int(to), ctypes.c_int(seq))

    def kv_row(self, il, seq, pos, k=True):
        nb = int(self.L.or_model_kv_row_bytes(_P(self.h)))
        p = self.L.or_model_kv_row(_P(self.h), ctypes.c_int(il), ctypes.c_int(seq), ctypes.c_int(pos),
                                   ctypes.c_int(1 if k else 0))
        return np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_int8)), shape=(nb,)).copy()


def ref_available():
    return os.path.exists(REF_PATH)


class Ref(_Common):
    """The reference's own hot path, compiled from its sources (oracle/_ref)."""
    prefix = "ref_"

    def __init__(self):
        if not os.path.exists(REF_PATH):
            raise RuntimeError(f"{REF_PATH} not built")
        L = self.lib = ctypes.CDLL(REF_PATH)
        L.ref_quantize_i8.restype = ctypes.c_float
        L.ref_dot_f32.restype = ctypes.c_float
        L.ref_vec_dot.restype = ctypes.c_float
        L.ref_weight_new.restype = _P
        L.ref_weight_new.argtypes = [ctypes.c_int, _P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.ref_model_open.restype = _P
        L.ref_model_open.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_char_p,
                                     ctypes.c_int]
        L.ref_isa.restype = ctypes.c_char_p
        if hasattr(L, "ref_sampler_new"):
            L.ref_sampler_new.restype = _P
            L.ref_sampler_new.argtypes = [_P, ctypes.c_int, ctypes.c_uint64, ctypes.c_int]
            L.ref_sampler_free.argtypes = [_P]
            L.ref_sampler_accept.argtypes = [_P, ctypes.c_int32]
            L.ref_sampler_distribution.argtypes = [_P, _P, ctypes.c_int, _P, _P, ctypes.c_int]
            L.ref_sampler_sample.restype = ctypes.c_int32
            L.ref_sampler_sample.argtypes = [_P, _P, ctypes.c_int]
            L.ref_sampler_draw.restype = ctypes.c_int32
            L.ref_sampler_draw.argtypes = [_P, _P, _P, ctypes.c_int]
            L.ref_sampler_verify.restype = ctypes.c_int32
            L.ref_sampler_verify.argtypes = [_P, _P, _P, ctypes.c_int, _P, _P, ctypes.c_int, ctypes.c_int32, _P]

    def cpu_ok(self):
        return bool(self.lib.ref_cpu_ok())

    def physical_cores(self):
        return int(self.lib.ref_physical_cores())

    def cpu_model(self):
        b = ctypes.create_string_buffer(256)
        self.lib.ref_cpu_model(b, 256)
        return b.value.decode()

    def set_threads(self, n):
        self.lib.ref_set_threads(ctypes.c_int(n))

    def matmul_rows(self, t, w, rows, cols, x=None, xq=None, n=1):
        """The reference's matmul over an unpacked weight: its row path (quant.cpp:330-351)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        x = np.zeros((n, cols), np.float32) if x is None else np.ascontiguousarray(x, dtype=np.float32)
        xq = np.zeros(n * (cols // 32), BLOCK_Q8) if xq is None else np.ascontiguousarray(xq, dtype=BLOCK_Q8)
        h = self.lib.ref_weight_new(t, ptr(w), rows, cols, 0)
        y = np.zeros((n, rows), dtype=np.float32)
        self.lib.ref_weight_matmul(_P(h), ptr(x), ptr(xq), ctypes.c_int(n), ptr(y))
        self.lib.ref_weight_free(_P(h))
        return y

    def matmul(self, t, w, rows, cols, xq, mode=1):
        """mode 1: compact panels; 2: compact + wide (as the engine packs them, engine.cpp:130-145)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        xq = np.ascontiguousarray(xq, dtype=BLOCK_Q8)
        n = xq.size // (cols // 32)
        h = self.lib.ref_weight_new(t, ptr(w), rows, cols, mode)
        y = np.zeros((n, rows), dtype=np.float32)
        x = np.zeros((n, cols), dtype=np.float32)  # unused by quantized weights
        self.lib.ref_weight_matmul(_P(h), ptr(x), ptr(xq), ctypes.c_int(n), ptr(y))
        self.lib.ref_weight_free(_P(h))
        return y

    def sampler(self, seed, penalties=True, **params):
        return RefSampler(self, seed, penalties, **params)

    def model(self, path, n_ctx, n_seq=1, wide=True, no_pack=False):
        """no_pack: the reference's MALKIN_NO_PACK (model.cpp:136): no panels, every matmul on the row path."""
        return RefModel(self, path, n_ctx, n_seq, (1 if wide else 0) | (2 if no_pack else 0))


class RefModel(_ModelBase):
    def __init__(self, r, path, n_ctx, n_seq, wide):
        self.L = r.lib
        self.errbuf = ctypes.create_string_buffer(512)
        self.h = self.L.ref_model_open(path.encode(), n_ctx, n_seq, int(wide), self.errbuf, 512)
        if not self.h:
            raise RuntimeError(self._err())
        c = (ctypes.c_int * 8)()
        self.L.ref_model_config(_P(self.h), c)
        self.cfg = dict(n_layer=c[0], n_embd=c[1], n_ff=c[2], n_head=c[3], n_head_kv=c[4], head_dim=c[5],
                        n_vocab=c[6])

    def close(self):
        if self.h:
            self.L.ref_model_free(_P(self.h))
            self.h = None

    __del__ = close

    def forward_batch(self, batch):
        batch = np.ascontiguousarray(batch, dtype=BATCH_TOKEN)
        nl = int((batch["logits"] != 0).sum())
        logits = np.zeros((max(nl, 1), self.cfg["n_vocab"]), dtype=np.float32)
        rc = self.L.ref_model_forward_batch(_P(self.h), ptr(batch), ctypes.c_int(len(batch)), ptr(logits),
                                            self.errbuf, 512)
        if rc != 0:
            raise RuntimeError(self._err())
        return logits[:nl]

    def forward(self, tokens, pos, all_logits=False, parent=None, seq=0):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        logits = np.zeros((n if all_logits else 1, self.cfg["n_vocab"]), dtype=np.float32)
        par = None if parent is None else np.ascontiguousarray(parent, dtype=np.int32)
        rc = self.L.ref_model_forward(_P(self.h), ptr(tokens), ctypes.c_int(n), ctypes.c_int(pos), ptr(logits),
                                      ctypes.c_int(1 if all_logits else 0), ptr(par), ctypes.c_int(seq), self.errbuf,
                                      512)
        if rc != 0:
            raise RuntimeError(self._err())
        return logits

    def move_kv(self, frm, to, seq=0):
        self.L.ref_model_move_kv(_P(self.h), ctypes.c_int(frm), ctypes.c_int(to), ctypes.c_int(seq))


class RefSampler:
    """The reference's own Sampler (sampler.cpp, compiled into oracle/_ref) behind OracleSampler's methods."""

    def __init__(self, r, seed, penalties=True, **params):
        self.r = r
        p = dict(SAMPLING_DEFAULTS, **params)
        pf = np.array([p["temperature"], p["top_p"], p["min_p"], p["presence"], p["frequency"]], np.float32)
        self.h = r.lib.ref_sampler_new(ptr(pf), p["top_k"], seed, 1 if penalties else 0)

    def close(self):
        if self.h:
            self.r.lib.ref_sampler_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def accept(self, tok):
        self.r.lib.ref_sampler_accept(self.h, int(tok))

    def distribution(self, logits):
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        probs = np.zeros(logits.size, np.float32)
        ids = np.zeros(logits.size, np.int32)
        n = self.r.lib.ref_sampler_distribution(self.h, ptr(logits), logits.size, ptr(probs), ptr(ids), logits.size)
        return [(float(probs[i]), int(ids[i])) for i in range(n)]

    def draw(self, d):
        pp, pi = _dist_arrays(d)
        return int(self.r.lib.ref_sampler_draw(self.h, ptr(pp), ptr(pi), len(pp)))

    def sample(self, logits):
        return int(self.r.lib.ref_sampler_sample(self.h, ptr(logits), logits.size))

    def verify(self, p, q, draft):
        pp, pi = _dist_arrays(p)
        qp, qi = _dist_arrays(q) if q else (np.zeros(1, np.float32), np.zeros(1, np.int32))
        a = ctypes.c_int()
        t = self.r.lib.ref_sampler_verify(self.h, ptr(pp), ptr(pi), len(pp), ptr(qp), ptr(qi), len(q), draft,
                                          ctypes.byref(a))
        return int(t), bool(a.value)
