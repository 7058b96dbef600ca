"""Kernel-level parity: every gfx950 kernel, called through the C ABI, against the CPU oracle and the golden vectors
written by the reference's own compiled code. Integer and byte work must be bit-exact, and so is every fp32 output:
the kernels reproduce the reference's rounding steps one for one."""
import ctypes

import numpy as np
import pytest

import malkin_amd as mk_
from malkin_amd import MkWeight
from oracle import bind

pytestmark = pytest.mark.gpu

L = mk_.load


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32)


def row_bytes(t, k):
    return bind.row_size(t, k)


def test_device_is_gfx950(mk):
    print("device", mk.device_name)
    assert mk.device_name.startswith("gfx950")


@pytest.mark.parametrize("t,rows,k", [(mk_.Q8_0, 24, 512), (mk_.Q8_0, 8, 96), (mk_.Q4_K, 16, 512),
                                      (mk_.Q6_K, 24, 768)])
def test_pack_roundtrip(mk, t, rows, k):
    import make_golden
    rng = np.random.default_rng(rows * k + t)
    w = make_golden.random_rows(rng, t, rows, k)
    src = mk.to_device(w)
    pb = L().mk_packed_bytes(t, rows, k)
    assert pb == w.nbytes
    packed = mk.alloc(pb)
    mk_.check(L().mk_pack_weight(mk.h, t, src.ptr, row_bytes(t, k), rows, k, packed.ptr))
    back = mk.alloc(w.nbytes)
    mk_.check(L().mk_unpack_weight(mk.h, t, packed.ptr, rows, k, back.ptr))
    assert np.array_equal(back.download(np.uint8), w.reshape(-1))
    assert not np.array_equal(packed.download(np.uint8), w.reshape(-1))  # the layout really changes


def test_quantize_q8(mk, golden, oracle):
    g = golden("quant.npz")
    x = g["x"]
    dx = mk.to_device(x)
    out = mk.alloc(x.size // 32 * 40)
    mk_.check(L().mk_quantize_q8(mk.h, dx.ptr, x.shape[0], x.shape[1], out.ptr))
    assert np.array_equal(out.download(np.uint8), g["q8"].reshape(-1))
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((64, 4096)) * 3).astype(np.float32)
    dx = mk.to_device(x)
    out = mk.alloc(x.size // 32 * 40)
    mk_.check(L().mk_quantize_q8(mk.h, dx.ptr, 64, 4096, out.ptr))
    assert np.array_equal(out.download(np.uint8), oracle.quantize_row_q8(x).view(np.uint8).reshape(-1))


def test_quantize_i8(mk, golden):
    g = golden("quant.npz")
    xi = g["xi"]
    dx = mk.to_device(xi)
    q = mk.alloc(xi.size)
    d = mk.alloc(4 * xi.shape[0])
    mk_.check(L().mk_quantize_i8(mk.h, dx.ptr, xi.shape[0], xi.shape[1], q.ptr, d.ptr))
    assert np.array_equal(q.download(np.int8).reshape(xi.shape), g["qi"])
    assert np.array_equal(bits(d.download(np.float32)), bits(g["di"]))


def test_silu(mk, golden):
    g = golden("quant.npz")
    dg, du = mk.to_device(g["g"]), mk.to_device(g["u"])
    mk_.check(L().mk_silu_mul(mk.h, g["g"].size, dg.ptr, du.ptr))
    assert np.array_equal(bits(dg.download(np.float32)), bits(g["silu"]))


# (rows, F): part of one workgroup per row, a row ending in a partial workgroup, a Qwen3-14B-wide row
@pytest.mark.parametrize("rows,F", [(5, 512), (3, 1056), (2, 17408)])
def test_silu_mul_q8(mk, oracle, rows, F):
    """Fused silu_mul + quantize of [gate | up] rows against the oracle, and of the same rows interleaved by 4."""
    rng = np.random.default_rng(2 + F)
    gu = rng.uniform(-20, 20, (rows, 2 * F)).astype(np.float32)
    dgu = mk.to_device(gu)
    out = mk.alloc(rows * F // 32 * 40)
    mk_.check(L().mk_silu_mul_q8(mk.h, dgu.ptr, rows, F, 0, out.ptr))
    exp = np.stack([oracle.silu_mul(r[:F], r[F:]) for r in gu])
    assert np.array_equal(out.download(np.uint8), oracle.quantize_row_q8(exp).view(np.uint8).reshape(-1))
    # the same rows with gate/up interleaved by 4
    gi = interleave4(gu[:, :F], gu[:, F:])
    dgi = mk.to_device(gi)
    out2 = mk.alloc(rows * F // 32 * 40)
    mk_.check(L().mk_silu_mul_q8(mk.h, dgi.ptr, rows, F, 1, out2.ptr))
    assert np.array_equal(out2.download(np.uint8), out.download(np.uint8))


def interleave4(gate, up):
    """[.., F] gate and up -> [.., 2F] rows interleaved by 4: 4 gate values, then the 4 up values of the same outputs."""
    lead = gate.shape[:-1]
    g4 = gate.reshape(*lead, -1, 4)
    u4 = up.reshape(*lead, -1, 4)
    return np.concatenate([g4, u4], axis=-1).reshape(*lead, -1)


@pytest.mark.parametrize("n", [16, 64, 2560, 4096, 5120, 8176, 8192])
def test_rmsnorm(mk, oracle, n):
    rng = np.random.default_rng(3 + n)
    rows = 7
    x = (rng.standard_normal((rows, n)) * 5).astype(np.float32)
    x[2] = 0.0  # zero row: scale from eps alone, Q8 blocks with d = 0
    x[4, : n // 2] *= 1e-30  # tiny values next to ordinary ones
    w = rng.uniform(0.5, 1.5, n).astype(np.float32)
    dx, dw = mk.to_device(x), mk.to_device(w)
    y = mk.alloc(x.nbytes)
    mk_.check(L().mk_rmsnorm(mk.h, dx.ptr, dw.ptr, rows, n, ctypes.c_float(1e-6), y.ptr))
    exp = np.stack([oracle.rmsnorm(r, w, 1e-6) for r in x])
    assert np.array_equal(bits(y.download(np.float32).reshape(rows, n)), bits(exp))
    if n % 32:
        return
    idx = np.array([6, 0, 2, 4, 3], np.int32)
    didx = mk.to_device(idx)
    out = mk.alloc(len(idx) * n // 32 * 40)
    mk_.check(L().mk_rmsnorm_q8(mk.h, dx.ptr, didx.ptr, dw.ptr, len(idx), n, ctypes.c_float(1e-6), out.ptr))
    assert np.array_equal(out.download(np.uint8), oracle.quantize_row_q8(exp[idx]).view(np.uint8).reshape(-1))


def _packed(mk, t, w, rows, k):
    src = mk.to_device(w)
    packed = mk.alloc(L().mk_packed_bytes(t, rows, k))
    mk_.check(L().mk_pack_weight(mk.h, t, src.ptr, row_bytes(t, k), rows, k, packed.ptr))
    return packed


def _matmul(mk, t, packed, rows, k, xq, n, wide, y=None, accumulate=False):
    dxq = mk.to_device(xq)
    if y is None:
        y = mk.alloc(n * rows * 4)
    wt = MkWeight(t, 1 if wide else 0, rows, k, packed.p)
    mk_.check(L().mk_matmul(mk.h, ctypes.byref(wt), dxq.ptr, n, y.ptr, rows, 1 if accumulate else 0))
    return y


def test_matmul_golden(mk, golden):
    g = golden("gemm.npz")
    cases = sorted({key.split("_")[0] for key in g.files})
    done = 0
    for c in cases:
        t = int(g[f"{c}_type"])
        if t not in (mk_.Q8_0, mk_.Q4_K, mk_.Q6_K):
            continue
        w = g[f"{c}_w"]
        rows = w.shape[0]
        k = (w.shape[1] // 34) * 32 if t == mk_.Q8_0 else (w.shape[1] // {12: 144, 14: 210}[t]) * 256
        packed = _packed(mk, t, w, rows, k)
        for key in g.files:
            if key.startswith(c + "_n") and key.endswith("_xq"):
                n = int(key[len(c) + 2:-3])
                xq = g[key]
                for wide, suffix in ((True, "_y"), (False, "_y_compact")):
                    y = _matmul(mk, t, packed, rows, k, xq, n, wide).download(np.float32).reshape(n, rows)
                    assert np.array_equal(bits(y), bits(g[f"{c}_n{n}{suffix}"])), (c, n, wide)
                    done += 1
    assert done >= 20


LARGE = [(t, n, 256, 4096) for t in (mk_.Q8_0, mk_.Q4_K, mk_.Q6_K) for n in (1, 3, 8, 17)] + [
    (mk_.Q8_0, 1, 65536, 1024),   # 2048 row groups of 32: the wide-workgroup shape
    (mk_.Q8_0, 8, 256, 12288),    # down-projection depth: several LDS chunks per row
    (mk_.Q6_K, 8, 256, 17408),
    (mk_.Q4_K, 2, 512, 17408),
    (mk_.Q8_0, 256, 512, 4096),   # int8-MFMA prefill GEMM, 32-token tiles (the grid fits the CUs once), 16 stages
    (mk_.Q8_0, 256, 4608, 256),   # 64-token tiles, 144 workgroups: the 6-stage ring
    (mk_.Q8_0, 131, 256, 2560),   # token tail inside a wave tile
    (mk_.Q8_0, 40, 96, 512),      # a full and a half-height row tile: the plain tile order
    (mk_.Q8_0, 24, 64, 416),      # 13 blocks: a partial last K stage
    (mk_.Q8_0, 70, 32, 96),       # one half-height row tile, a single short K stage, two token tiles
    (mk_.Q8_0, 9, 1024, 256),     # short-batch kernel, K split: 64 row tiles, 7 idle token columns
    (mk_.Q8_0, 100, 160, 1024),   # a full and a quarter-height 128-row tile; second token tile 36 tokens
    (mk_.Q8_0, 65, 1120, 320),    # 9 row tiles (plain order), 10 blocks: a 2-block last K stage
    # K-quant int8-MFMA GEMM (n > 32): partial row tiles, several token tiles, XCD-mapped grids, 1..4 ring cycles;
    # the 5..32-token cases go to the short-batch kernels (K split over four waves up to 8192 rows)
    (mk_.Q4_K, 9, 128, 512),
    (mk_.Q4_K, 100, 160, 1024),
    (mk_.Q4_K, 64, 1024, 1536),
    (mk_.Q4_K, 9, 6144, 256),     # 384 K-split row tiles
    (mk_.Q6_K, 9, 128, 512),
    (mk_.Q6_K, 9, 6144, 256),     # n <= 16: compact arithmetic
    (mk_.Q6_K, 16, 6176, 512),    # 386 row tiles: two workgroups per CU
    (mk_.Q6_K, 17, 6144, 512),    # the tree-verify batch size: wide arithmetic, two token tiles
    (mk_.Q6_K, 17, 1024, 1024),   # ... on fewer rows
    (mk_.Q6_K, 100, 160, 2560),
]


@pytest.mark.parametrize("t,n,rows,k", LARGE)
def test_matmul_large_vs_oracle(mk, oracle, t, n, rows, k):
    """Real widths, several LDS chunks, both workgroup shapes, and the residual-accumulate epilogue."""
    import make_golden
    rng = np.random.default_rng(100 * t + n + rows + k)
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    packed = _packed(mk, t, w, rows, k)
    exp = oracle.matmul(t, w, rows, k, xq.reshape(-1), wide=True)
    y = _matmul(mk, t, packed, rows, k, xq.view(np.uint8), n, True).download(np.float32).reshape(n, rows)
    assert np.array_equal(bits(y), bits(exp))
    base = rng.standard_normal((n, rows)).astype(np.float32)
    yd = mk.to_device(base)
    _matmul(mk, t, packed, rows, k, xq.view(np.uint8), n, True, y=yd, accumulate=True)
    assert np.array_equal(bits(yd.download(np.float32).reshape(n, rows)), bits(base + exp))


@pytest.mark.parametrize("t,n,rows,k", [(mk_.Q8_0, 40, 96, 512), (mk_.Q8_0, 3, 64, 256)])
def test_matmul_strided_output(mk, oracle, t, n, rows, k):
    """y at a 4-byte offset with an odd token stride: the GEMM's scalar store path and the GEMV's strided stores."""
    import make_golden
    rng = np.random.default_rng(11 * n + rows)
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    packed = _packed(mk, t, w, rows, k)
    exp = oracle.matmul(t, w, rows, k, xq.reshape(-1), wide=True)
    ys = rows + 3
    base = rng.standard_normal(n * ys + 1).astype(np.float32)
    yd = mk.to_device(base)
    dxq = mk.to_device(xq.view(np.uint8))
    wt = MkWeight(t, 1, rows, k, packed.p)
    mk_.check(L().mk_matmul(mk.h, ctypes.byref(wt), dxq.ptr, n, ctypes.c_void_p(yd.p + 4), ys, 1))
    got = yd.download(np.float32)
    want = base.copy()
    view = want[1:].reshape(n, ys)
    view[:, :rows] += exp
    assert np.array_equal(bits(got), bits(want))


@pytest.mark.parametrize("t,n,rows,k", [(mk_.Q6_K, 40, 160, 1024), (mk_.Q6_K, 33, 64, 512), (mk_.Q4_K, 40, 64, 512)])
def test_matmul_compact_batches(mk, oracle, t, n, rows, k):
    """wide = 0 (MALKIN_NO_WIDE): the compact arithmetic at every batch size, through the K-quant GEMM."""
    import make_golden
    rng = np.random.default_rng(5 * n + rows + t)
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    packed = _packed(mk, t, w, rows, k)
    exp = oracle.matmul(t, w, rows, k, xq.reshape(-1), wide=False)
    y = _matmul(mk, t, packed, rows, k, xq.view(np.uint8), n, False).download(np.float32).reshape(n, rows)
    assert np.array_equal(bits(y), bits(exp))


# Short batches (5..32 tokens) on the MFMA short-batch kernels: one wave per 16-row tile on matrices of more than
# 8192 rows (and on Q4_K above 16 tokens), four waves splitting each stage's K units otherwise; one or two 16-token
# tiles, token tails inside a tile, the wide and compact Q6_K arithmetic.
SHORT = [
    (mk_.Q8_0, 5, 8224, 256), (mk_.Q8_0, 23, 8224, 512),         # one wave per tile, one and two token tiles
    (mk_.Q4_K, 12, 8224, 512), (mk_.Q4_K, 20, 8224, 512), (mk_.Q4_K, 20, 256, 1024),
    (mk_.Q6_K, 12, 8224, 512), (mk_.Q6_K, 20, 8224, 512),
    (mk_.Q8_0, 6, 96, 2048), (mk_.Q8_0, 30, 160, 1024),           # K split over four waves
    (mk_.Q4_K, 7, 64, 1536), (mk_.Q4_K, 16, 192, 512),
    (mk_.Q6_K, 13, 96, 1024), (mk_.Q6_K, 25, 64, 512), (mk_.Q6_K, 32, 4096, 256),
    (mk_.Q4_K, 3, 8224, 512), (mk_.Q4_K, 4, 8224, 256), (mk_.Q8_0, 3, 24576, 256),  # 3-4 tokens on many rows
    (mk_.Q6_K, 5, 96, 512), (mk_.Q8_0, 8, 4096, 1024), (mk_.Q4_K, 6, 2048, 2048),  # up to 8 tokens: two units a tile
    (mk_.Q6_K, 17, 16384, 512), (mk_.Q4_K, 17, 16384, 256),   # K-quant GEMM at 17 tokens: padding elements skipped
    # K split, two token tiles in 20 token slots (17..20 tokens): every count, both grid shapes; 21 tokens: 32 slots
    (mk_.Q6_K, 18, 2048, 512), (mk_.Q6_K, 19, 4096, 256), (mk_.Q6_K, 20, 96, 1024), (mk_.Q6_K, 21, 160, 512),
    (mk_.Q8_0, 20, 160, 512), (mk_.Q8_0, 19, 4096, 256), (mk_.Q8_0, 17, 5120, 512),
    # 4 tokens on 2048..8192 rows: the K-split pairs (chain waves); 12 tokens: Q6_K on eight term waves
    (mk_.Q4_K, 4, 2048, 1024), (mk_.Q6_K, 4, 5120, 512), (mk_.Q8_0, 4, 8192, 256), (mk_.Q6_K, 12, 320, 1024),
    # K split past 8192 rows: up to 8 tokens (17408 rows of K-quants, 12288 of Q8_0), Q6_K at 17..32 tokens
    (mk_.Q4_K, 8, 8224, 512), (mk_.Q6_K, 4, 17408, 256), (mk_.Q8_0, 6, 12288, 256), (mk_.Q6_K, 18, 8224, 256),
    # pairs on 16-unit stages (K a multiple of 512) and on 8-unit ones (768)
    (mk_.Q6_K, 8, 64, 768), (mk_.Q4_K, 3, 8224, 768), (mk_.Q8_0, 7, 2048, 1536),
    # K-quant GEMM past one 128-row tile per CU: a full tile per CU plus 32-row tail tiles (8, 64 and 256 of them)
    (mk_.Q6_K, 17, 33024, 256), (mk_.Q4_K, 20, 34816, 256), (mk_.Q6_K, 32, 40960, 256),
]


@pytest.mark.parametrize("t,n,rows,k", SHORT)
def test_matmul_short_batches(mk, oracle, t, n, rows, k):
    """The short-batch kernels bit for bit against the oracle, both Q6_K arithmetics, and the accumulate epilogue."""
    import make_golden
    print("short batch", dict(t=t, n=n, rows=rows, k=k), flush=True)
    rng = np.random.default_rng(7 * t + n + rows + k)
    w = make_golden.random_rows(rng, t, rows, k)
    x = rng.uniform(-2, 2, (n, k)).astype(np.float32)
    xq = oracle.quantize_row_q8(x)
    packed = _packed(mk, t, w, rows, k)
    for wide in ((True, False) if t == mk_.Q6_K else (True,)):
        exp = oracle.matmul(t, w, rows, k, xq.reshape(-1), wide=wide)
        y = _matmul(mk, t, packed, rows, k, xq.view(np.uint8), n, wide).download(np.float32).reshape(n, rows)
        assert np.array_equal(bits(y), bits(exp)), wide
        base = rng.standard_normal((n, rows)).astype(np.float32)
        yd = mk.to_device(base)
        _matmul(mk, t, packed, rows, k, xq.view(np.uint8), n, wide, y=yd, accumulate=True)
        assert np.array_equal(bits(yd.download(np.float32).reshape(n, rows)), bits(base + exp)), wide


F32_CASES = [(t, n, rows, k) for t in (mk_.Q8_0, mk_.Q4_K, mk_.Q6_K) for n in (1, 2) for rows, k in ((64, 256), (96, 4096))] + [
    (mk_.Q8_0, 1, 512, 8192),    # widest fused row: two 16-value chunks per thread
    (mk_.Q8_0, 2, 48, 2560),     # a width that is not a multiple of 256
    (mk_.Q6_K, 1, 40, 12288 // 2),
]


@pytest.mark.parametrize("t,n,rows,k", F32_CASES)
def test_matmul_f32_matches_unfused(mk, oracle, t, n, rows, k):
    """mk_matmul_f32 (rmsnorm / quantization inside the matmul) == mk_rmsnorm_q8 / mk_quantize_q8 + mk_matmul, and
    both == the oracle."""
    import make_golden
    rng = np.random.default_rng(7 * t + 3 * n + rows + k)
    w = make_golden.random_rows(rng, t, rows, k)
    packed = _packed(mk, t, w, rows, k)
    stride = k + 32  # a token stride wider than the row
    x = np.zeros((n, stride), np.float32)
    x[:, :k] = (rng.standard_normal((n, k)) * 3).astype(np.float32)
    if n == 2:
        x[1, :k] = 0.0  # zero row: rmsnorm scale from eps alone, d = 0 blocks
    nw = rng.uniform(0.5, 1.5, k).astype(np.float32)
    dx, dnw = mk.to_device(x), mk.to_device(nw)
    wt = MkWeight(t, 1, rows, k, packed.p)
    for norm in (True, False):
        xq = mk.alloc(n * k // 32 * 40)
        if norm:
            for i in range(n):
                mk_.check(L().mk_rmsnorm_q8(mk.h, ctypes.c_void_p(dx.p + i * stride * 4), None, dnw.ptr, 1, k,
                                            ctypes.c_float(1e-6), ctypes.c_void_p(xq.p + i * (k // 32) * 40)))
        else:
            for i in range(n):
                mk_.check(L().mk_quantize_q8(mk.h, ctypes.c_void_p(dx.p + i * stride * 4), 1, k,
                                             ctypes.c_void_p(xq.p + i * (k // 32) * 40)))
        base = rng.standard_normal((n, rows)).astype(np.float32)
        y_ref = mk.to_device(base)
        mk_.check(L().mk_matmul(mk.h, ctypes.byref(wt), xq.ptr, n, y_ref.ptr, rows, 1))
        y = mk.to_device(base)
        mk_.check(L().mk_matmul_f32(mk.h, ctypes.byref(wt), dx.ptr, stride, dnw.ptr if norm else None,
                                    ctypes.c_float(1e-6), n, y.ptr, rows, 1, 0))
        got, exp = y.download(np.float32), y_ref.download(np.float32)
        assert np.array_equal(bits(got), bits(exp)), (norm, t, n, rows, k)
        # and the unfused path against the oracle
        xs = np.stack([oracle.rmsnorm(x[i, :k], nw, 1e-6) if norm else x[i, :k] for i in range(n)])
        oq = oracle.quantize_row_q8(xs)
        assert np.array_equal(xq.download(np.uint8), oq.view(np.uint8).reshape(-1))
        ref = oracle.matmul(t, w, rows, k, oq.reshape(-1), wide=True)
        assert np.array_equal(bits(got.reshape(n, rows)), bits(base + ref))


@pytest.mark.parametrize("t,n,F,k", [(mk_.Q8_0, 1, 96, 4096), (mk_.Q8_0, 2, 64, 512), (mk_.Q4_K, 1, 64, 2048),
                                     (mk_.Q6_K, 2, 32, 1024)])
def test_matmul_f32_silu_pairs(mk, oracle, t, n, F, k):
    """Gate/up rows interleaved by 4 with the silu epilogue == the plain matmul of the same rows, then the oracle's
    silu_mul (kernels_avx512.cpp:271-280) on the de-interleaved gate and up."""
    import make_golden
    rng = np.random.default_rng(11 * t + n + F + k)
    gate = make_golden.random_rows(rng, t, F, k)
    up = make_golden.random_rows(rng, t, F, k)
    rows = np.concatenate([np.concatenate([gate[4 * j:4 * j + 4], up[4 * j:4 * j + 4]]) for j in range(F // 4)])
    packed = _packed(mk, t, rows, 2 * F, k)
    x = (rng.standard_normal((n, k)) * 2).astype(np.float32)
    nw = rng.uniform(0.5, 1.5, k).astype(np.float32)
    dx, dnw = mk.to_device(x), mk.to_device(nw)
    wt = MkWeight(t, 1, 2 * F, k, packed.p)
    h = mk.alloc(n * F * 4)
    mk_.check(L().mk_matmul_f32(mk.h, ctypes.byref(wt), dx.ptr, k, dnw.ptr, ctypes.c_float(1e-6), n, h.ptr, F, 0, 1))
    gu = mk.alloc(n * 2 * F * 4)
    mk_.check(L().mk_matmul_f32(mk.h, ctypes.byref(wt), dx.ptr, k, dnw.ptr, ctypes.c_float(1e-6), n, gu.ptr, 2 * F,
                                0, 0))
    gu = gu.download(np.float32).reshape(n, F // 4, 8)
    g_, u_ = gu[:, :, :4].reshape(n, F), gu[:, :, 4:].reshape(n, F)
    exp = np.stack([oracle.silu_mul(g_[i], u_[i]) for i in range(n)])
    assert np.array_equal(bits(h.download(np.float32).reshape(n, F)), bits(exp))
    # accumulate with the silu epilogue is refused
    rc = L().mk_matmul_f32(mk.h, ctypes.byref(wt), dx.ptr, k, None, ctypes.c_float(0), n, h.ptr, F, 1, 1)
    assert rc == mk_.MK_ERR_INVALID


def test_matmul_f32_unsupported(mk):
    wt = MkWeight(mk_.Q8_0, 0, 8, 64, None)
    rc = L().mk_matmul_f32(mk.h, ctypes.byref(wt), None, 64, None, ctypes.c_float(0), 3, None, 8, 0, 0)
    assert rc == mk_.MK_ERR_UNSUPPORTED
    assert b"no fused kernel" in L().mk_last_error()


def test_attend_gqa_golden(mk, golden):
    g = golden("attention.npz")
    for i in range(int(g["count"])):
        G, D, n, ne, stride = (int(v) for v in g[f"a{i}_meta"])
        dq, dk, dv = mk.to_device(g[f"a{i}_q"]), mk.to_device(g[f"a{i}_k"]), mk.to_device(g[f"a{i}_v"])
        dex = mk.to_device(g[f"a{i}_extra"]) if ne else None
        out = mk.alloc(G * D * 4)
        scale = np.float32(1.0) / np.sqrt(np.float32(D))
        mk_.check(L().mk_attend_gqa(mk.h, dq.ptr, G, D, dk.ptr, dv.ptr, stride, D + 4, n, ctypes.c_float(scale),
                                    out.ptr, dex.ptr if dex else None, ne))
        assert np.array_equal(bits(out.download(np.float32)), bits(g[f"a{i}_out"])), (G, D, n)


def test_argmax_top2(mk, oracle):
    rng = np.random.default_rng(4)
    rows, V = 6, 151936
    l = rng.standard_normal((rows, V)).astype(np.float32)
    l[1, [5, 70000, 151935]] = 99.0      # ties: first index wins
    l[2, :] = 1.0                       # all equal
    l[3, 151935] = 50.0                 # max at the end
    l[4, [0, 1]] = 40.0
    dl = mk.to_device(l)
    t1, t2 = mk.alloc(rows * 4), mk.alloc(rows * 4)
    mk_.check(L().mk_argmax_top2(mk.h, dl.ptr, rows, V, t1.ptr, t2.ptr))
    a, b = t1.download(np.int32), t2.download(np.int32)
    for r in range(rows):
        assert (a[r], b[r]) == oracle.top2(l[r]), r
        assert a[r] == oracle.argmax(l[r])


@pytest.mark.parametrize("t", [mk_.Q8_0, mk_.Q4_K, mk_.Q6_K, mk_.F32])
def test_dequantize_rows(mk, oracle, t):
    import make_golden
    rng = np.random.default_rng(t)
    k = 512
    if t == mk_.F32:
        w = rng.standard_normal((10, k)).astype(np.float32).view(np.uint8).reshape(10, -1)
    else:
        w = make_golden.random_rows(rng, t, 10, k)
    ids = np.array([3, 0, 9, 3], np.int32)
    dw, di = mk.to_device(w), mk.to_device(ids)
    out = mk.alloc(len(ids) * k * 4)
    mk_.check(L().mk_dequantize_rows(mk.h, t, dw.ptr, w.shape[1], di.ptr, len(ids), k, out.ptr))
    exp = np.stack([oracle.dequantize_row(t, w[i], k) for i in ids])
    assert np.array_equal(bits(out.download(np.float32).reshape(len(ids), k)), bits(exp))


def test_errors_are_statuses(mk):
    wt = MkWeight(1, 0, 8, 64, None)  # F16: no device kernel
    rc = L().mk_matmul(mk.h, ctypes.byref(wt), None, 1, None, 8, 0)
    assert rc == mk_.MK_ERR_INVALID
    assert b"no kernel" in L().mk_last_error()
    rc = L().mk_silu_mul(mk.h, 17, None, None)
    assert rc == mk_.MK_ERR_UNSUPPORTED


def _kv_perm(D):
    """Element e of a K row sits at byte D/16 * (e % 16) + e // 16 of the device cache's permuted row."""
    e = np.arange(D)
    return (D // 16) * (e % 16) + e // 16


# (D, H, KV, token seqs, token key counts, n_ctx): the multi-row kernel for plain batches of 16+ tokens, and the
# per-token kernel past its LDS limit.
ROWS_CASES = [
    (128, 32, 8, [0] * 64, [600 + t + 1 for t in range(64)], 700),                  # prefill continuation, G = 4
    (64, 8, 2, [0] * 13 + [1] * 24, [40 + t for t in range(13)] + [5 + t for t in range(24)], 64),  # mixed blocks
    (128, 16, 1, [1] * 20, [t + 1 for t in range(20)], 32),                           # G = 16: one token per block
    (128, 5, 1, [0] * 17, [100 + 3 * t for t in range(17)], 160),                     # G = 5: 15 rows per block
    (64, 4, 4, [t % 3 for t in range(40)], [1 + t for t in range(40)], 48),          # G = 1, 3 sequences per block
    (128, 8, 4, [0] * 16, [1840 - t for t in range(16)], 1840),                       # longest rows in LDS
    (128, 8, 4, [0] * 16, [1900 - t for t in range(16)], 1900),                       # per-token kernel
    (96, 4, 2, [0, 1, 0], [33, 17, 50], 64),                                          # other head size: generic
    (64, 20, 1, [0, 0], [10, 30], 32),                                                # G = 20: generic
]


def _check_q8_variant(mk, oracle, call, got):
    """call(out, xq) runs the _q8 variant of the attention call that produced got ([n][H*D] fp32): its out must equal
    got bit for bit and its xq the oracle's quantize_acts of got (quant.h:11-16 blocks) byte for byte."""
    n, k = got.shape
    out2, xq = mk.alloc(n * k * 4), mk.alloc(n * k // 32 * 40)
    call(out2.ptr, xq.ptr)
    assert np.array_equal(bits(out2.download(np.float32).reshape(n, k)), bits(got))
    assert np.array_equal(xq.download(np.uint8), oracle.quantize_row_q8(got).view(np.uint8).reshape(-1))


@pytest.mark.parametrize("case", range(len(ROWS_CASES)))
def test_attention_batch_vs_oracle(mk, oracle, case):
    D, H, KV, seqs, nks, n_ctx = ROWS_CASES[case]
    G, n, n_seq = H // KV, len(seqs), max(seqs) + 1
    print("attention case", case, dict(D=D, H=H, KV=KV, n=n), flush=True)
    rng = np.random.default_rng(300 + case)
    k8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    v8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    q = rng.standard_normal((n, H * D)).astype(np.float32)
    dk = mk.to_device(np.ascontiguousarray(k8[..., np.argsort(_kv_perm(D))]))
    dv, dks, dvs, dq = mk.to_device(v8), mk.to_device(ks), mk.to_device(vs), mk.to_device(q)
    dseq, dnk = mk.to_device(np.array(seqs, np.int32)), mk.to_device(np.array(nks, np.int32))
    out = mk.alloc(n * H * D * 4)
    kv = mk_.MkKvCache(dk.ptr, dv.ptr, dks.ptr, dvs.ptr, 1, n_seq, KV, D, n_ctx)
    mk_.check(L().mk_attention(mk.h, dq.ptr, H * D, out.ptr, H * D, n, H, ctypes.byref(kv), 0, dseq.ptr, dnk.ptr,
                               None, None, max(nks)))
    got = out.download(np.float32).reshape(n, H * D)
    _check_q8_variant(mk, oracle, lambda o, x: mk_.check(L().mk_attention_q8(
        mk.h, dq.ptr, H * D, o, H * D, n, H, ctypes.byref(kv), 0, dseq.ptr, dnk.ptr, None, None, max(nks), x)), got)
    # The reference's KV rows: KV heads x D int8, then KV float scales (model.cpp:105-110).
    row = KV * D + 4 * KV
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    for s in sorted(set(seqs)):
        kb = np.zeros((n_ctx, row), np.uint8)
        vb = np.zeros((n_ctx, row), np.uint8)
        kb[:, :KV * D] = k8[s].transpose(1, 0, 2).reshape(n_ctx, KV * D).view(np.uint8)
        vb[:, :KV * D] = v8[s].transpose(1, 0, 2).reshape(n_ctx, KV * D).view(np.uint8)
        kb[:, KV * D:] = ks[s].T.copy().view(np.uint8).reshape(n_ctx, 4 * KV)
        vb[:, KV * D:] = vs[s].T.copy().view(np.uint8).reshape(n_ctx, 4 * KV)
        kf, vf = kb.reshape(-1), vb.reshape(-1)
        for t in (t for t in range(n) if seqs[t] == s):
            for g in range(KV):
                exp = oracle.attend_gqa(q[t, g * G * D:(g + 1) * G * D], G, D, kf[g * D:], vf[g * D:], row,
                                        (KV - g) * D + 4 * g, nks[t], scale)
                assert np.array_equal(bits(got[t, g * G * D:(g + 1) * G * D]), bits(exp)), (case, t, g)


# (D, H, KV, token seqs, positions, n_ctx, max_keys): the fused decode kernel against the two-launch path.
DECODE_CASES = [
    (128, 32, 8, [0], [575], 640, 640),              # decode step of the north-star shape, G = 4
    (128, 32, 8, [0, 2, 1], [5, 900, 301], 1024, 1000),  # three sequences, three slot counts' worth of keys
    (64, 8, 2, [1, 0], [0, 63], 64, 64),             # D = 64 (a pair's RoPE partner in another lane), first position
    (128, 40, 8, [0], [129], 256, 256),              # G = 5
    (128, 32, 8, [0], [10], 4096, 4096),             # beyond the LDS capacity: MK_ERR_UNSUPPORTED
]


@pytest.mark.parametrize("case", range(len(DECODE_CASES)))
def test_attention_decode_fused(mk, oracle, case):
    """mk_attention_decode == mk_qk_norm_rope_kv + mk_attention: outputs bit for bit, every cache byte identical."""
    D, H, KV, seqs, pos, n_ctx, max_keys = DECODE_CASES[case]
    n, n_seq = len(seqs), max(seqs) + 1
    print("decode case", case, dict(D=D, H=H, KV=KV, n=n, max_keys=max_keys), flush=True)
    rng = np.random.default_rng(500 + case)
    QKV = (H + 2 * KV) * D
    qkv = rng.standard_normal((n, QKV)).astype(np.float32)
    norms = rng.uniform(0.5, 1.5, 2 * D).astype(np.float32)
    ang = np.arange(n_ctx, dtype=np.float32)[:, None] * np.float32(1e-3) * (np.arange(D // 2, dtype=np.float32) + 1)
    cos_t, sin_t = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    k8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    v8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    ksc = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    vsc = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    meta = {name: mk.to_device(np.array(v, np.int32)) for name, v in
            (("rpos", pos), ("seq", seqs), ("kv_row", pos), ("n_keys", [p + 1 for p in pos]))}
    dnorm, dcos, dsin = mk.to_device(norms), mk.to_device(cos_t), mk.to_device(sin_t)

    def cache():
        bufs = [mk.to_device(k8), mk.to_device(v8), mk.to_device(ksc), mk.to_device(vsc)]
        return bufs, mk_.MkKvCache(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, 1, n_seq, KV, D, n_ctx)

    eps = ctypes.c_float(1e-6)
    # two launches (q, k written in place)
    ba, kva = cache()
    dqa, outa = mk.to_device(qkv), mk.alloc(n * H * D * 4)
    mk_.check(L().mk_qk_norm_rope_kv(mk.h, dqa.ptr, dqa.offset(H * D * 4), dqa.offset((H + KV) * D * 4), QKV, n, H,
                                     dnorm.ptr, dnorm.offset(D * 4), eps, dcos.ptr, dsin.ptr, meta["rpos"].ptr,
                                     meta["seq"].ptr, meta["kv_row"].ptr, ctypes.byref(kva), 0))
    mk_.check(L().mk_attention(mk.h, dqa.ptr, QKV, outa.ptr, H * D, n, H, ctypes.byref(kva), 0, meta["seq"].ptr,
                               meta["n_keys"].ptr, None, None, max_keys))
    # fused
    bb, kvb = cache()
    dqb, outb = mk.to_device(qkv), mk.alloc(n * H * D * 4)
    rc = L().mk_attention_decode(mk.h, dqb.ptr, QKV, n, H, dnorm.ptr, dnorm.offset(D * 4), eps, dcos.ptr, dsin.ptr,
                                 meta["rpos"].ptr, meta["seq"].ptr, meta["kv_row"].ptr, meta["n_keys"].ptr,
                                 ctypes.byref(kvb), 0, outb.ptr, H * D, max_keys)
    if max_keys >= 4096:
        assert rc == mk_.MK_ERR_UNSUPPORTED
        return
    mk_.check(rc)
    assert np.array_equal(bits(outa.download(np.float32)), bits(outb.download(np.float32)))
    for x, y in zip(ba, bb):
        assert np.array_equal(x.download(np.uint8), y.download(np.uint8))
    assert np.array_equal(dqb.download(np.float32), qkv.reshape(-1))  # raw projections untouched
    # the _q8 variant on a third copy of the cache: same out, same cache bytes, and the BlockQ8 rows of out
    bc, kvc = cache()
    _check_q8_variant(mk, oracle, lambda o, x: mk_.check(L().mk_attention_decode_q8(
        mk.h, dqb.ptr, QKV, n, H, dnorm.ptr, dnorm.offset(D * 4), eps, dcos.ptr, dsin.ptr, meta["rpos"].ptr,
        meta["seq"].ptr, meta["kv_row"].ptr, meta["n_keys"].ptr, ctypes.byref(kvc), 0, o, H * D, max_keys, x)),
        outb.download(np.float32).reshape(n, H * D))
    for x, y in zip(ba, bc):
        assert np.array_equal(x.download(np.uint8), y.download(np.uint8))


# Rows longer than one workgroup's LDS (about 11600 keys at D = 128, 7600 at D = 64): scores in global slots of the
# context's scratch. (D, H, KV, token seqs, n_keys, n_ctx, ancestors per token)
LONG_CASES = [
    (128, 8, 2, [0], [12200], 12200, None),                                   # a decode step, G = 4
    (128, 4, 4, [0, 1, 0], [12000, 9000, 11000], 12100, None),               # G = 1, two sequences
    (64, 4, 2, [0, 0], [16500, 16400], 16500, None),                         # D = 64
    (128, 8, 2, [0, 0, 0], [12000, 12000, 12000], 12100, [[], [12001], [12001, 12003]]),  # a tree past the prefix
]


def _tree(P, depth):
    """Ancestor rows of the engine's tree after a P-token prefix: node 0 at row P, chain / alternative of depth k at
    rows P + 1 + 2k and P + 2 + 2k, both children of the chain node of depth k - 1 (of node 0 for k = 0); a node's
    list runs from node 0 down to itself."""
    par = [-1] + [0 if k == 0 else 2 * k - 1 for k in range(depth) for _ in range(2)]
    out = []
    for t in range(len(par)):
        chain, u = [], t
        while u >= 0:
            chain.append(P + u)
            u = par[u]
        out.append(chain[::-1])
    return out


# The grouped kernel (all G query heads of a KV group per workgroup, G = 2..5, D = 128): trees, and keys past the
# decode and multi-row kernels' LDS, where one workgroup per (token, head) would take more than one round of the
# 256 CUs. (D, H, KV, token seqs, n_keys, n_ctx, ancestors per token)
GRP_CASES = [
    (128, 40, 8, [0] * 17, [2048] * 17, 2100, _tree(2048, 8)),              # config 5's verification tree, G = 5
    (128, 16, 8, [0] * 17, [2000] * 17, 2048, _tree(2000, 8)),              # the same tree at G = 2
    (128, 12, 4, [0] * 11 + [1] * 11, [1500] * 11 + [1300] * 11, 1600,
     _tree(1500, 5) + _tree(1300, 5)),                                      # G = 3, two sequences' trees
    (128, 32, 8, [0] * 9, [1200] * 9, 1300, _tree(1200, 4)),                # G = 4
    (128, 40, 8, [0] * 20, [2000 - t for t in range(20)], 2048, None),     # 20 plain tokens past the multi-row LDS
    (128, 40, 8, [0], [2048], 2048, None),                                  # one head per workgroup: a long decode
    (128, 16, 8, [0, 0, 0], [9000] * 3, 9100, [[9000], [9000, 9001], [9000, 9002]]),  # past the per-head fp32 tiles
]


@pytest.mark.parametrize("case", range(len(LONG_CASES)))
def test_attention_long_rows_vs_oracle(mk, oracle, case):
    _attention_vs_oracle(mk, oracle, LONG_CASES[case], 700 + case, "long attention case %d" % case, True)


@pytest.mark.parametrize("case", range(len(GRP_CASES)))
def test_attention_grouped_vs_oracle(mk, oracle, case):
    _attention_vs_oracle(mk, oracle, GRP_CASES[case], 800 + case, "grouped attention case %d" % case, False)


def _attention_vs_oracle(mk, oracle, spec, seed, name, long_rows):
    D, H, KV, seqs, nks, n_ctx, ancs = spec
    G, n, n_seq = H // KV, len(seqs), max(seqs) + 1
    print(name, dict(D=D, H=H, KV=KV, n=n, keys=max(nks)), flush=True)
    rng = np.random.default_rng(seed)
    k8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    v8 = rng.integers(-127, 128, (n_seq, KV, n_ctx, D), dtype=np.int8)
    ks = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    vs = rng.uniform(0.001, 0.05, (n_seq, KV, n_ctx)).astype(np.float32)
    q = (rng.standard_normal((n, H * D)) * 3).astype(np.float32)
    dk = mk.to_device(np.ascontiguousarray(k8[..., np.argsort(_kv_perm(D))]))
    dv, dks, dvs, dq = mk.to_device(v8), mk.to_device(ks), mk.to_device(vs), mk.to_device(q)
    dseq, dnk = mk.to_device(np.array(seqs, np.int32)), mk.to_device(np.array(nks, np.int32))
    anc_off = anc = None
    max_keys = max(nks)
    if ancs is not None:
        off = np.cumsum([0] + [len(a) for a in ancs]).astype(np.int32)
        flat = np.array([r for a in ancs for r in a] or [0], np.int32)
        anc_off, anc = mk.to_device(off), mk.to_device(flat)
        max_keys = max(nk + len(a) for nk, a in zip(nks, ancs))
    out = mk.alloc(n * H * D * 4)
    kv = mk_.MkKvCache(dk.ptr, dv.ptr, dks.ptr, dvs.ptr, 1, n_seq, KV, D, n_ctx)
    need = L().mk_attention_scratch_bytes(D, max_keys, n * H)
    assert (need > 0) == long_rows  # global slots only past one workgroup's LDS
    if need:
        mk_.check(L().mk_reserve_scratch(mk.h, need))
    mk_.check(L().mk_attention(mk.h, dq.ptr, H * D, out.ptr, H * D, n, H, ctypes.byref(kv), 0, dseq.ptr, dnk.ptr,
                               anc_off.ptr if anc_off is not None else None, anc.ptr if anc is not None else None,
                               max_keys))
    got = out.download(np.float32).reshape(n, H * D)
    _check_q8_variant(mk, oracle, lambda o, x: mk_.check(L().mk_attention_q8(
        mk.h, dq.ptr, H * D, o, H * D, n, H, ctypes.byref(kv), 0, dseq.ptr, dnk.ptr,
        anc_off.ptr if anc_off is not None else None, anc.ptr if anc is not None else None, max_keys, x)), got)
    row = KV * D + 4 * KV
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    for s in sorted(set(seqs)):
        kb = np.zeros((n_ctx, row), np.uint8)
        vb = np.zeros((n_ctx, row), np.uint8)
        kb[:, :KV * D] = k8[s].transpose(1, 0, 2).reshape(n_ctx, KV * D).view(np.uint8)
        vb[:, :KV * D] = v8[s].transpose(1, 0, 2).reshape(n_ctx, KV * D).view(np.uint8)
        kb[:, KV * D:] = ks[s].T.copy().view(np.uint8).reshape(n_ctx, 4 * KV)
        vb[:, KV * D:] = vs[s].T.copy().view(np.uint8).reshape(n_ctx, 4 * KV)
        kf, vf = kb.reshape(-1), vb.reshape(-1)
        for t in (t for t in range(n) if seqs[t] == s):
            extra = np.array(ancs[t], np.int32) if ancs is not None and ancs[t] else None
            for g in range(KV):
                exp = oracle.attend_gqa(q[t, g * G * D:(g + 1) * G * D], G, D, kf[g * D:], vf[g * D:], row,
                                        (KV - g) * D + 4 * g, nks[t], scale, extra=extra)
                assert np.array_equal(bits(got[t, g * G * D:(g + 1) * G * D]), bits(exp)), (name, t, g)


def test_attention_long_rows_need_scratch():
    """Rows whose global slot does not fit the context's scratch (a fresh context holds 1 MiB: 131072 keys' slot)
    fail with a status, nothing launched."""
    c = mk_.Context(0)
    try:
        D, KV, n_ctx = 128, 1, 140000
        buf = mk_.load()
        dk = c.alloc(KV * n_ctx * D)
        ds = c.alloc(KV * n_ctx * 4)
        dq = c.alloc(D * 4)
        dseq = c.to_device(np.zeros(1, np.int32))
        dnk = c.to_device(np.array([n_ctx], np.int32))
        out = c.alloc(D * 4)
        kv = mk_.MkKvCache(dk.ptr, dk.ptr, ds.ptr, ds.ptr, 1, 1, KV, D, n_ctx)
        rc = buf.mk_attention(c.h, dq.ptr, D, out.ptr, D, 1, 1, ctypes.byref(kv), 0, dseq.ptr, dnk.ptr, None, None,
                              n_ctx)
        assert rc == mk_.MK_ERR_INVALID and b"scratch" in buf.mk_last_error()
    finally:
        c.close()
