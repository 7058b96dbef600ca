// Load-time repack of GGUF rows into the CDNA layout of layout.h (and the inverse, for round-trip tests).
// Replaces the reference's VNNI panel packing (gemm_avx512.cpp:376-505, quant.cpp:212-229): same information, laid
// out for 128-byte-coalesced wavefront streams instead of 16-row AVX-512 panels. Runs on the device, once per weight.
#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

__device__ __forceinline__ void copy_bytes(uint8_t* d, const uint8_t* s, int n) {
  for (int i = 0; i < n; ++i) d[i] = s[i];
}

// GGUF Q6_K: 6-bit value k (0..255) of a 210-byte super-block (quant.cpp:108-128 layout).
__device__ __forceinline__ int q6_value(const uint8_t* s, int k) {
  const int n = k >> 7, rem = k & 127, c = rem >> 5, l = rem & 31;
  const uint8_t lo = s[64 * n + l + (c & 1) * 32];
  const int nib = c >= 2 ? lo >> 4 : lo & 0xF;
  const int hb = (s[128 + 32 * n + l] >> (2 * c)) & 3;
  return nib | (hb << 4);
}

template <bool kPack>
__global__ void k_q8_0(uint8_t* gguf, size_t srb, uint8_t* dst, int64_t rows, int64_t nb, int64_t r0, int64_t nrows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * nb) return;
  const int64_t lr = i / nb, r = r0 + lr, b = i % nb, g = r / 8;
  const int rr = (int)(r % 8);
  const PackedQ8_0 L{rows, nb};
  uint8_t* row = gguf + lr * srb + b * 34;  // GGUF block (source when packing, destination when unpacking)
  uint8_t* lo = dst + L.quants(g, b) + rr * 16;
  uint8_t* sc = dst + L.scales(g, b) + rr * 2;
  if (kPack) {
    copy_bytes(sc, row, 2);
    copy_bytes(lo, row + 2, 16);
    copy_bytes(lo + 128, row + 18, 16);
  } else {
    copy_bytes(row, sc, 2);
    copy_bytes(row + 2, lo, 16);
    copy_bytes(row + 18, lo + 128, 16);
  }
}

template <bool kPack>
__global__ void k_q4_k(uint8_t* gguf, size_t srb, uint8_t* dst, int64_t rows, int64_t nsb, int64_t r0, int64_t nrows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * nsb) return;
  const int64_t lr = i / nsb, r = r0 + lr, sb = i % nsb, g = r / 8;
  const int rr = (int)(r % 8);
  const PackedQ4_K L{rows, nsb};
  uint8_t* blk = gguf + lr * srb + sb * 144;
  uint8_t* hdr = dst + L.headers(g, sb) + rr * 16;
  if (kPack)
    copy_bytes(hdr, blk, 16);
  else
    copy_bytes(blk, hdr, 16);
  for (int j2 = 0; j2 < 4; ++j2) {
    uint8_t* q = dst + L.quants(g, sb, j2) + rr * 16;
    if (kPack) {
      copy_bytes(q, blk + 16 + 32 * j2, 16);
      copy_bytes(q + 128, blk + 16 + 32 * j2 + 16, 16);
    } else {
      copy_bytes(blk + 16 + 32 * j2, q, 16);
      copy_bytes(blk + 16 + 32 * j2 + 16, q + 128, 16);
    }
  }
}

__global__ void k_pack_q6_k(const uint8_t* __restrict__ src, size_t srb, uint8_t* __restrict__ dst, int64_t rows,
                            int64_t nsb, int64_t r0, int64_t nrows) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nrows * nsb) return;
  const int64_t lr = i / nsb, r = r0 + lr, sb = i % nsb, g = r / 8;
  const int rr = (int)(r % 8);
  const PackedQ6_K L{rows, nsb};
  const uint8_t* s = src + lr * srb + sb * 210;
  for (int b8 = 0; b8 < 8; ++b8) {
    uint8_t* nib = dst + L.quants(g, sb, b8) + rr * 16;
    uint8_t* hb = dst + L.quants(g, sb, b8) + 128 + rr * 8;
    uint8_t h[8] = {0};
    for (int l = 0; l < 16; ++l) {
      const int a = q6_value(s, 32 * b8 + l), b = q6_value(s, 32 * b8 + 16 + l);
      nib[l] = (uint8_t)((a & 0xF) | ((b & 0xF) << 4));
    }
    for (int w = 0; w < 2; ++w)
      for (int m = 0; m < 4; ++m)
        for (int ii = 0; ii < 4; ++ii) h[4 * w + ii] |= (uint8_t)((q6_value(s, 32 * b8 + 16 * w + 4 * m + ii) >> 4) << (2 * m));
    copy_bytes(hb, h, 8);
  }
  copy_bytes(dst + L.scales(g, sb) + rr * 16, s + 192, 16);
  copy_bytes(dst + L.dscale(g, sb) + rr * 2, s + 208, 2);
}

__global__ void k_unpack_q6_k(const uint8_t* __restrict__ packed, uint8_t* __restrict__ dst, size_t drb, int64_t rows,
                              int64_t nsb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * nsb) return;
  const int64_t r = i / nsb, sb = i % nsb, g = r / 8;
  const int rr = (int)(r % 8);
  const PackedQ6_K L{rows, nsb};
  uint8_t* s = dst + r * drb + sb * 210;
  uint8_t q[256];
  for (int b8 = 0; b8 < 8; ++b8) {
    const uint8_t* nib = packed + L.quants(g, sb, b8) + rr * 16;
    const uint8_t* hb = packed + L.quants(g, sb, b8) + 128 + rr * 8;
    for (int k = 0; k < 32; ++k) {
      const int l = k & 15, w = k >> 4, m = (k & 15) >> 2, ii = k & 3;
      const int low = (k < 16 ? nib[l] : nib[l] >> 4) & 0xF;
      const int high = (hb[4 * w + ii] >> (2 * m)) & 3;
      q[32 * b8 + k] = (uint8_t)(low | (high << 4));
    }
  }
  for (int n = 0; n < 2; ++n)
    for (int l = 0; l < 32; ++l) {
      const int q1 = q[128 * n + l], q2 = q[128 * n + 32 + l], q3 = q[128 * n + 64 + l], q4 = q[128 * n + 96 + l];
      s[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
      s[64 * n + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
      s[128 + 32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
    }
  copy_bytes(s + 192, packed + L.scales(g, sb) + rr * 16, 16);
  copy_bytes(s + 208, packed + L.dscale(g, sb) + rr * 2, 2);
}

int blocks_for(int64_t n, int t) { return (int)((n + t - 1) / t); }

}  // namespace

size_t packed_bytes(int type, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0 || rows % kRowGroup) return 0;
  switch (type) {
    case kQ8_0:
      return cols % 32 ? 0 : PackedQ8_0{rows, cols / 32}.bytes();
    case kQ4_K:
      return cols % 256 ? 0 : PackedQ4_K{rows, cols / 256}.bytes();
    case kQ6_K:
      return cols % 256 ? 0 : PackedQ6_K{rows, cols / 256}.bytes();
    default:
      return 0;
  }
}

static size_t gguf_row_bytes(int type, int64_t cols) {
  switch (type) {
    case kQ8_0:
      return (size_t)(cols / 32) * 34;
    case kQ4_K:
      return (size_t)(cols / 256) * 144;
    case kQ6_K:
      return (size_t)(cols / 256) * 210;
    default:
      return 0;
  }
}

void pack_weight_rows(hipStream_t s, int type, const void* src, size_t srb, int64_t r0, int64_t nrows, int64_t rows,
                      int64_t cols, void* dst) {
  if (!packed_bytes(type, rows, cols)) throw Error(MK_ERR_UNSUPPORTED, "pack_weight: no CDNA layout for this type/shape");
  require(r0 >= 0 && nrows >= 0 && r0 % kRowGroup == 0 && (nrows % kRowGroup == 0 || r0 + nrows == rows) &&
              r0 + nrows <= rows,
          "pack_weight: row range outside the weight or not on 8-row groups");
  if (nrows == 0) return;
  auto* in = const_cast<uint8_t*>(static_cast<const uint8_t*>(src));
  auto* out = static_cast<uint8_t*>(dst);
  const int T = 256;
  switch (type) {
    case kQ8_0:
      hipLaunchKernelGGL(k_q8_0<true>, dim3(blocks_for(nrows * (cols / 32), T)), dim3(T), 0, s, in, srb, out, rows,
                         cols / 32, r0, nrows);
      break;
    case kQ4_K:
      hipLaunchKernelGGL(k_q4_k<true>, dim3(blocks_for(nrows * (cols / 256), T)), dim3(T), 0, s, in, srb, out, rows,
                         cols / 256, r0, nrows);
      break;
    case kQ6_K:
      hipLaunchKernelGGL(k_pack_q6_k, dim3(blocks_for(nrows * (cols / 256), T)), dim3(T), 0, s, in, srb, out, rows,
                         cols / 256, r0, nrows);
      break;
  }
  check_launch("pack_weight");
}

void pack_weight(hipStream_t s, int type, const void* src, size_t srb, int64_t rows, int64_t cols, void* dst) {
  pack_weight_rows(s, type, src, srb, 0, rows, rows, cols, dst);
}

void unpack_weight(hipStream_t s, int type, const void* packed, int64_t rows, int64_t cols, void* dst) {
  if (!packed_bytes(type, rows, cols)) throw Error(MK_ERR_UNSUPPORTED, "unpack_weight: no CDNA layout for this type/shape");
  const size_t drb = gguf_row_bytes(type, cols);
  const int T = 256;
  // The Q8_0 / Q4_K kernels move bytes in both directions: their first pointer is the GGUF side.
  switch (type) {
    case kQ8_0:
      hipLaunchKernelGGL(k_q8_0<false>, dim3(blocks_for(rows * (cols / 32), T)), dim3(T), 0, s,
                         static_cast<uint8_t*>(dst), drb, const_cast<uint8_t*>(static_cast<const uint8_t*>(packed)),
                         rows, cols / 32, (int64_t)0, rows);
      break;
    case kQ4_K:
      hipLaunchKernelGGL(k_q4_k<false>, dim3(blocks_for(rows * (cols / 256), T)), dim3(T), 0, s,
                         static_cast<uint8_t*>(dst), drb, const_cast<uint8_t*>(static_cast<const uint8_t*>(packed)),
                         rows, cols / 256, (int64_t)0, rows);
      break;
    case kQ6_K:
      hipLaunchKernelGGL(k_unpack_q6_k, dim3(blocks_for(rows * (cols / 256), T)), dim3(T), 0, s,
                         static_cast<const uint8_t*>(packed), static_cast<uint8_t*>(dst), drb, rows, cols / 256);
      break;
  }
  check_launch("unpack_weight");
}

}  // namespace mk
