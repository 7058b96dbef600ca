"""Parity at the full sizes of BASELINE.json's kernel-level configurations, through the C ABI:

  config 1  one Q8_0 GEMM, W 9728x2560, X 512x2560 quantized by the reference routine (the int8 MFMA prefill kernel);
  config 2  decode GEMV over the Qwen3-14B FFN shapes (gate/up 5120->17408, down 17408->5120) in Q4_K and Q6_K at
            n = 1, 4, 8.

Weights as BASELINE.json draws them: entries N(0, 0.02), quantized by the GGUF writer's quantizer (synth.quantize_rows,
the reference's quantize_row_* restated); activations N(0, 1) through the reference's Q8_0 activation quantizer.

Every output is compared with a float64 product of the dequantized operands under the reference's own criterion
(|y - y64| / rms(y64) < 1e-5, test_quant.cpp:250-256), which catches any misplaced row, token or block; a spread of
rows (the first and last tiles included) is compared bit for bit with the CPU oracle over the full depth."""
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


def device_matmul(mk, t, w, rows, k, xq, n):
    src = mk.to_device(w)
    packed = mk.alloc(L().mk_packed_bytes(t, rows, k))
    mk_.check(L().mk_pack_weight(mk.h, t, src.ptr, bind.row_size(t, k), rows, k, packed.ptr))
    dxq = mk.to_device(xq)
    y = mk.alloc(n * rows * 4)
    wt = MkWeight(t, 1, rows, k, packed.p)
    mk_.check(L().mk_matmul(mk.h, ctypes.byref(wt), dxq.ptr, n, y.ptr, rows, 0))
    return y.download(np.float32).reshape(n, rows)


def dequantized(oracle, t, w, k):
    return np.stack([oracle.dequantize_row(t, r, k) for r in w]).astype(np.float64)


def acts64(xq):
    return (xq["d"].astype(np.float64)[..., None] * xq["qs"].astype(np.float64)).reshape(xq.shape[0], -1)


def spread(rows, step):
    return np.unique(np.concatenate([np.arange(0, rows, step), np.arange(rows - 48, rows)]))


def check(oracle, t, w, k, xq, y, sel, wide=True):
    exp = oracle.matmul(t, w[sel], len(sel), k, xq.reshape(-1), wide=wide)
    assert np.array_equal(bits(y[:, sel]), bits(exp))
    y64 = acts64(xq) @ dequantized(oracle, t, w, k).T
    rel = np.abs(y.astype(np.float64) - y64).max() / np.sqrt(np.mean(y64 ** 2))
    assert rel < 1e-5, rel


def normal_rows(synth_lib, rng, t, rows, k):
    """BASELINE.json's weights: entries N(0, 0.02), quantized to type t by the GGUF writer's quantizer."""
    return synth_lib.quantize_rows(t, (rng.standard_normal((rows, k), dtype=np.float32) * np.float32(0.02)))


def test_config1_gemm_q8_0_full(mk, oracle, synth_lib):
    rows, k, n = 9728, 2560, 512
    print("config 1 GEMM", rows, k, n, flush=True)
    rng = np.random.default_rng(9728)
    w = normal_rows(synth_lib, rng, mk_.Q8_0, rows, k)
    xq = oracle.quantize_row_q8(rng.standard_normal((n, k)).astype(np.float32))
    y = device_matmul(mk, mk_.Q8_0, w, rows, k, xq.view(np.uint8), n)
    check(oracle, mk_.Q8_0, w, k, xq, y, spread(rows, 97))


@pytest.mark.parametrize("t", [mk_.Q4_K, mk_.Q6_K])
@pytest.mark.parametrize("rows,k", [(17408, 5120), (5120, 17408)])
def test_config2_gemv_full(mk, oracle, synth_lib, t, rows, k):
    rng = np.random.default_rng(t * 100 + rows)
    w = normal_rows(synth_lib, rng, t, rows, k)
    for n in (1, 4, 8):
        print("config 2 GEMV", t, rows, k, n, flush=True)
        xq = oracle.quantize_row_q8(rng.standard_normal((n, k)).astype(np.float32))
        y = device_matmul(mk, t, w, rows, k, xq.view(np.uint8), n)
        check(oracle, t, w, k, xq, y, spread(rows, 211))
