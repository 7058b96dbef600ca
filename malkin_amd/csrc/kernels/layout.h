// CDNA weight layout ("packed" weights), shared by the repack, GEMV and GEMM kernels.
//
// Rows are taken in groups of 8 (all Qwen3 matmul row counts are multiples of 8). Within a group, each row's bytes
// for one work unit are split into 16-byte planes stored row after row, so one wavefront instruction reads whole
// 128-byte lines: lane l of a wave reads 16 bytes at 16 * l of a plane. Scales live in a separate stream after the
// quants. Every format keeps the GGUF byte count (34 / 144 / 210 bytes per 32 / 256 / 256 weights).
//
//  Q8_0 (unit = one 32-weight block b, nb = cols/32 units per row):
//    quants  [g][b]  : lo plane 8 rows x 16 B (qs 0..15), hi plane 8 rows x 16 B (qs 16..31)      256 B
//    scales  [g][b]  : 8 rows x f16 d                                                              16 B
//  Q4_K (unit = 64 weights = one 32-byte GGUF nibble chunk j2 of super-block sb; 4 units per sb):
//    quants  [g][sb][j2] : lo plane 8 x 16 B (chunk bytes 0..15), hi plane 8 x 16 B (bytes 16..31)  256 B
//    headers [g][sb] : 8 rows x 16 B GGUF header (f16 d, f16 dmin, 12 B packed 6-bit scales/mins)  128 B
//  Q6_K (unit = one 32-weight Q8 block b8 of super-block sb; 8 units per sb):
//    quants  [g][sb][b8] : nib plane 8 x 16 B, hbit plane 8 x 8 B                                  192 B
//        nib byte l (0..15) = low nibble of q[l] | low nibble of q[l+16] << 4  (q = 6-bit value, 0..63)
//        hbit word w (0..1), byte i (0..3), bits 2m..2m+1 = high 2 bits of q[16 w + 4 m + i]
//    scales  [g][sb] : 8 rows x 16 int8 sub-block scales                                           128 B
//    d       [g][sb] : 8 rows x f16 d                                                              16 B
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mk {

enum : int { kF32 = 0, kF16 = 1, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14, kBF16 = 30 };
constexpr int kRowGroup = 8;

struct PackedQ8_0 {
  int64_t rows, nb;
  __host__ __device__ size_t quants(int64_t g, int64_t b) const { return (size_t)(g * nb + b) * 256; }
  __host__ __device__ size_t scales(int64_t g, int64_t b) const {
    return (size_t)(rows / 8) * nb * 256 + (size_t)(g * nb + b) * 16;
  }
  __host__ __device__ size_t bytes() const { return (size_t)rows * nb * 34; }
};

struct PackedQ4_K {
  int64_t rows, nsb;
  __host__ __device__ size_t quants(int64_t g, int64_t sb, int j2) const {
    return ((size_t)(g * nsb + sb) * 4 + j2) * 256;
  }
  __host__ __device__ size_t headers(int64_t g, int64_t sb) const {
    return (size_t)(rows / 8) * nsb * 1024 + (size_t)(g * nsb + sb) * 128;
  }
  __host__ __device__ size_t bytes() const { return (size_t)rows * nsb * 144; }
};

struct PackedQ6_K {
  int64_t rows, nsb;
  __host__ __device__ size_t quants(int64_t g, int64_t sb, int b8) const {
    return ((size_t)(g * nsb + sb) * 8 + b8) * 192;
  }
  __host__ __device__ size_t scales(int64_t g, int64_t sb) const {
    return (size_t)(rows / 8) * nsb * 1536 + (size_t)(g * nsb + sb) * 128;
  }
  __host__ __device__ size_t dscale(int64_t g, int64_t sb) const {
    return (size_t)(rows / 8) * nsb * (1536 + 128) + (size_t)(g * nsb + sb) * 16;
  }
  __host__ __device__ size_t bytes() const { return (size_t)rows * nsb * 210; }
};

}  // namespace mk
