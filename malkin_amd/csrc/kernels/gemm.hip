// Prefill GEMM for Q8_0 weights on int8 MFMA (v_mfma_i32_32x32x32_i8), bit-identical to the reference's panel kernel
// (gemm_avx512.cpp:67-102):
//   y[t][r] = sum over blocks b, in order, of fma(float(int dot of block b), f16(dw[r][b]) * dx[t][b], acc).
// K = 32 of the MFMA is exactly one Q8_0 block, so every MFMA yields the exact int32 dots of one block for a 32 x 32
// (rows x tokens) tile, and the epilogue folds them into the fp32 chains with the reference's rounding. Per output and
// block that epilogue is a conversion, a scale product and an fma. On the VALU (4 cycles per wave instruction) those
// three cost 6x the int8 MFMA itself, so two of them run on the matrix cores instead:
//   conversion: the int8 MFMA starts from C = 0x4B400000, the bits of 12582912.0f = 1.5 * 2^23. |dot| <= 32 * 128 *
//     128 < 2^22 keeps the sum inside that binade, so its bits read as the float 12582912 + dot, and an fp32 MFMA
//     outer product adding (-12582912) * 1 to every element (v_mfma_f32_16x16x1_4b_f32, C = those bits) leaves
//     float(dot) exactly;
//   scale product: v_mfma_f32_32x32x1_2b_f32 with A = dw (one row per lane) and B = dx (one token per lane) yields
//     round(dw * dx) for a 32 x 64 tile, in the accumulator layout of the two int8 MFMAs; no other product is added
//     (K = 1), so the rounding is that of one fp32 multiply. A zero product may come out as +0 where the VALU gives
//     -0; the fma that consumes it returns the same value either way, because the chain never holds -0 (it starts at
//     +0 and an exact cancellation rounds to +0).
// That leaves one VALU fma per output and block.
//
// A workgroup owns a 128-row x TOK-token tile and walks the K dimension in stages of KB blocks held in a ring of NS
// LDS buffers; its wave w computes rows 32 (w % 4) .. + 31 and WT tokens of the tile. Three forms:
//   TOK = WT = 64, 4 waves, KB = 4 (26 KB per stage, 3 stages: two workgroups per CU; or 2 stages with one result
//     set, each step folding its own MFMA results: three workgroups per CU): a step is one block, its two int8 MFMAs
//     the two 32-token halves;
//   TOK = 64, WT = 32, 8 waves, KB = 8 (52 KB per stage, 3 stages: one workgroup per CU, two waves per SIMD): waves
//     w and w + 4 take the two 32-token halves of the same rows;
//   TOK = WT = 32, 4 waves, KB = 8 (43 KB per stage, 3 stages): for grids that fit the CUs once at 32 tokens.
// With WT = 32 a step is two blocks, its two int8 MFMAs one block each, both folding into the one accumulator in
// block order, and the scale-product MFMA's two halves are then the two blocks. A stage holds:
//   A  [KB][128 rows][32 B]  the rows' quants (from the CDNA planes of layout.h),
//   B  [KB][TOK tok][32 B]   the tokens' BlockQ8 quants,
//   dx [KB][TOK tok]  f32    activation scales,
//   dw [KB][128 rows] f16    weight scales.
// Rows of A and B are 32 bytes with their two 16-byte halves swapped on every other group of 8 rows, so the MFMA
// operand reads (lane l: row l % 32, half l / 32) hit distinct banks. All copies are direct global -> LDS loads
// (global_load_lds_dwordx4 / _dword: lane i of a wave instruction writes bytes [size * i, size * (i + 1)) after the
// instruction's LDS base), issued NS - 1 stages ahead, so the data of NS - 1 stages is in flight while a stage is
// computed and no register holds it on the way.
//
// Accumulator layout of v_mfma_i32_32x32x32_i8 (checked on gfx950): lane l, element i holds
//   row 8 * (i / 4) + 4 * (l / 32) + i % 4, column l % 32.
// v_mfma_f32_32x32x1_2b_f32 holds block j in elements 16 j .. 16 j + 15 in the same layout, block j taking A and B
// from lanes 32 j .. 32 j + 31 (checked on gfx950, together with the conversion and the product rounding).
#include <utility>

#include "ctx.h"
#include "ops.h"

namespace mk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

constexpr int kThreads = 256;
constexpr int kRowsT = 128;  // workgroup tile rows
constexpr int kMagic = 0x4B400000;       // bits of 12582912.0f
constexpr float kMagicF = 12582912.0f;

// Forms: TOK tokens per workgroup tile, WT tokens per wave (64: a step is one block, its two int8 MFMAs the two
// 32-token halves; 32: a step is two blocks), NW = 4 TOK / WT waves (wave w: rows 32 (w % 4), tokens WT (w / 4) of
// the tile), KB blocks per stage (four steps).
template <int TOK, int WT>
struct StageLds {
  static constexpr int NW = 4 * TOK / WT;              // waves
  static constexpr int KB = WT == 64 ? 4 : 8;          // blocks per stage
  static constexpr int a = 0;                          // KB * 128 * 32 bytes
  static constexpr int b = a + KB * kRowsT * 32;       // KB * TOK * 32
  static constexpr int dx = b + KB * TOK * 32;         // KB * TOK floats
  static constexpr int dw = dx + KB * TOK * 4;         // KB * 128 halves
  static constexpr int bytes = dw + KB * kRowsT * 2;
  // A pieces per wave and stage: its row group's 32 rows of blocks w / 4, w / 4 + NW / 4, ...
  static constexpr int apw = KB * 4 / NW;
  // copies per wave and stage: apw A pieces; TOK = 64: B halves 2, dx 1, dw 1 (block w); TOK = 32: B 2, dx 1 (both
  // blocks), dw 2 (blocks 2 w, 2 w + 1)
  static constexpr int loads = TOK == 64 ? apw + 4 : apw + 5;
};
static_assert(StageLds<64, 64>::KB == StageLds<64, 64>::NW && StageLds<64, 32>::KB == StageLds<64, 32>::NW &&
                  StageLds<32, 32>::KB == 2 * StageLds<32, 32>::NW,
              "one wave copies the B, dx and dw parts of KB / NW blocks");

// Byte offset of half h (0/1) of row r within a [rows][32 B] operand slab.
__device__ __forceinline__ int slab_off(int r, int h) { return r * 32 + ((h ^ ((r >> 3) & 1)) << 4); }

__device__ __forceinline__ void load_lds16(const void* g, uint8_t* l) { lds_copy16(g, l); }
// The ring's copies are tracked by vmcnt and waited for explicitly (the stage about to be computed only). Reads of a
// buffer finish before the barrier that precedes its next fill (lgkmcnt(0) before that barrier).

__device__ __forceinline__ void load_lds4(const void* g, uint8_t* l) { lds_copy4(g, l); }

// Waves per SIMD: a wave's MFMAs overlap the VALU work of another wave on its SIMD far better than its own (the step
// below, alone on a SIMD: 334 cycles; two waves: about 185 cycles per step and SIMD), so the TOK = 64 forms (two
// four-wave workgroups per CU, or one of eight waves) keep within 256 registers; TOK = 32 runs one wave per SIMD and
// keeps that wave's register budget.
// RA: how many steps ahead the operands are read from LDS (two where two waves share a SIMD: each wave then runs
// about half as fast and the other wave's reads queue in front of its own).
template <int TOK, int WT, int NS>
constexpr int gemm_waves() { return TOK == 64 ? (NS == 2 ? 3 : 2) : 1; }
template <int TOK, int WT, int NS, int RA>
__global__ __launch_bounds__((64 * StageLds<TOK, WT>::NW)) __attribute__((amdgpu_waves_per_eu(
    gemm_waves<TOK, WT, NS>(), gemm_waves<TOK, WT, NS>()))) void k_gemm_q8_0(const uint8_t* W, int64_t rows, int64_t cols,
                                                                       const BlockQ8* x, int n, float* __restrict__ y,
                                                                       int64_t ys, int accumulate, int n_rt, int n_tt,
                                                                       int vec) {
  using S = StageLds<TOK, WT>;
  constexpr int KB = S::KB;
  extern __shared__ __align__(16) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rg = w & 3, tw = WT * (w >> 2);  // wave w: rows 32 rg .. 32 rg + 31, tokens tw .. tw + WT - 1 of the tile
  // Workgroup -> (row tile, token tile): tiles numbered row-major, each XCD a contiguous run of them, so the token
  // tiles of a row tile share an XCD and its L2 holds the rows once.
  const int tile = xcd_run((int)blockIdx.x, n_rt * n_tt), rt = tile / n_tt, tt = tile % n_tt;
  const int nb = (int)(cols / 32);
  const PackedQ8_0 L{rows, nb};
  const int64_t g0 = (int64_t)rt * (kRowsT / 8);                  // first 8-row group of the tile
  const int ngroups = (int)min<int64_t>(kRowsT / 8, rows / 8 - g0);  // 4 .. 16 (rows % 32 == 0)
  // Waves whose 32 rows lie past the matrix (a partial last row tile) only copy in the three-per-CU form (NS = 2):
  // there the branch also lets the wave fit its 168 registers without spilling (5 spilled before; config 1 54.2 ->
  // 53.4 us, 24576 x 4096 at 512 tokens 180.1 -> 177.6, bit-identical); the other forms run 1-4 % slower with it.
  const bool live = NS != 2 || 32 * rg < 8 * ngroups;
  const int t0 = tt * TOK;
  const int nstages = (nb + KB - 1) / KB;

  // Copy mapping. Loads are never predicated: past the matrix they re-read valid data, unused.
  //   A: wave w copies the 32 rows of its row group rg, one 1 KB instruction per block (blocks w / 4 + k NW / 4):
  //      lane -> row 32 rg + lane / 2, physical half lane % 2 (logical half (lane % 2) ^ ((lane / 16) & 1)), 16 bytes
  //      of plane h of the row's group unit.
  //   B: TOK = 64: wave w copies block w, tokens 32 c + lane / 2 for c = 0, 1; TOK = 32: blocks 2 w and 2 w + 1,
  //      tokens lane / 2; the same half mapping, 16 qs bytes.
  //   dx: TOK = 64: block w, lane -> token lane; TOK = 32: lane -> block 2 w + lane / 32, token lane % 32.
  //   dw: block w (TOK = 32: blocks 2 w, 2 w + 1): lane -> the f16 scales of rows 2 lane, 2 lane + 1 (4 bytes of a
  //       group's 16-byte entry).
  // Addresses are a wave-uniform base that moves with the block plus a fixed 32-bit per-lane offset (the TOK = 32 dx
  // copy: its block, too, is per lane).
  const int a_row = 32 * rg + (lane >> 1);
  const int a_gi = min(a_row >> 3, ngroups - 1);
  const int half_sw = (lane & 1) ^ ((lane >> 4) & 1);
  const uint32_t a_off = (uint32_t)(a_gi * nb * 256 + (half_sw << 7) + (a_row & 7) * 16);
  const uint32_t b_off0 = (uint32_t)((min(t0 + (lane >> 1), n - 1) - t0) * nb * 40 + 8 + 16 * half_sw);
  const uint32_t b_off1 = (uint32_t)((min(t0 + 32 + (lane >> 1), n - 1) - t0) * nb * 40 + 8 + 16 * half_sw);
  const uint32_t dx_off = (uint32_t)((min(t0 + (TOK == 64 ? lane : lane & 31), n - 1) - t0) * nb * 40);
  const uint32_t dw_off = (uint32_t)(min(lane >> 2, ngroups - 1) * nb * 16 + 4 * (lane & 3));
  const uint8_t* a_base = W + L.quants(g0, 0);
  const uint8_t* x_base = reinterpret_cast<const uint8_t*>(x + (int64_t)t0 * nb);
  const uint8_t* dw_base = W + L.scales(g0, 0);
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // Copy I of stage sn into LDS buffer BUF; a stage is S::loads copies per wave: apw A pieces, then TOK = 64: B
  // halves 0 and 1, dx, dw; TOK = 32: B of blocks 2 w and 2 w + 1, dx, dw of blocks 2 w and 2 w + 1.
  const int wblk = wu >> 2, wrg = wu & 3;
  auto copy = [&]<int BUF, int I>(int sn) __attribute__((always_inline)) {
    uint8_t* st = smem + BUF * S::bytes;
    const int b0 = sn * KB;
    if constexpr (I < S::apw) {
      const int blk = wblk + I * (S::NW / 4);
      load_lds16(a_base + (size_t)min(b0 + blk, nb - 1) * 256 + a_off, st + S::a + blk * kRowsT * 32 + wrg * 1024);
    } else if constexpr (TOK == 64) {
      constexpr int J = I - S::apw;
      const int b = min(b0 + wu, nb - 1);
      if constexpr (J == 0)
        load_lds16(x_base + (size_t)b * 40 + b_off0, st + S::b + wu * TOK * 32);
      else if constexpr (J == 1)
        load_lds16(x_base + (size_t)b * 40 + b_off1, st + S::b + wu * TOK * 32 + 32 * 32);
      else if constexpr (J == 2)
        load_lds4(x_base + (size_t)b * 40 + dx_off, st + S::dx + wu * TOK * 4);
      else
        load_lds4(dw_base + (size_t)b * 16 + dw_off, st + S::dw + wu * kRowsT * 2);
    } else {
      constexpr int J = I - S::apw;
      if constexpr (J < 2) {
        const int b = min(b0 + 2 * wu + J, nb - 1);
        load_lds16(x_base + (size_t)b * 40 + b_off0, st + S::b + (2 * wu + J) * TOK * 32);
      } else if constexpr (J == 2) {
        const int bl = min(b0 + 2 * wu + (lane >> 5), nb - 1);  // per lane
        load_lds4(x_base + (size_t)bl * 40 + dx_off, st + S::dx + 2 * wu * TOK * 4);
      } else {
        const int b = min(b0 + 2 * wu + J - 3, nb - 1);
        load_lds4(dw_base + (size_t)b * 16 + dw_off, st + S::dw + (2 * wu + J - 3) * kRowsT * 2);
      }
    }
  };
  // Copies I0 .. I1 - 1 of stage sn into buffer BUF.
  auto copies = [&]<int BUF, int I0, int I1>(int sn) __attribute__((always_inline)) {
    [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
      (copy.template operator()<BUF, I0 + I>(sn), ...);
    }(std::make_integer_sequence<int, I1 - I0>{});
  };
  static_assert(S::loads == (TOK == 64 ? S::apw + 4 : S::apw + 5), "copies per wave and stage");
  // A whole stage (the ring's first fills).
  auto issue = [&]<int BUF>(int sn) __attribute__((always_inline)) { copies.template operator()<BUF, 0, S::loads>(sn); };

  v16f acc0 = {}, acc1 = {};  // WT = 64: tokens 0..31, 32..63; WT = 32: acc0 only
  v16i magic;
#pragma unroll
  for (int i = 0; i < 16; ++i) magic[i] = kMagic;
  asm volatile("" : "+v"(magic));  // keep it in VGPRs: as a uniform value it would be copied from SGPRs per MFMA
  const v32f zero = {};
  const int li = lane & 31, h = lane >> 5;
  const int arow = 32 * rg + li;
  // LDS byte offsets of this lane's operands within a stage buffer, block 0. The scale product's operands: WT = 64,
  // lane l: dw of row arow, dx of token l; WT = 32, lane l: block h (of the step's two): dw of row arow, dx of token
  // tw + li.
  const int off_a = S::a + slab_off(arow, h), off_b0 = S::b + slab_off(tw + li, h),
            off_b1 = S::b + slab_off(tw + 32 + li, h), off_dw = S::dw + 2 * arow + (WT == 64 ? 0 : h * kRowsT * 2),
            off_dx = S::dx + (WT == 64 ? 4 * lane : 4 * (tw + li) + h * TOK * 4);

  // Software pipeline over blocks j = 0, 1, ..., RA + 1 operand register sets and two result sets. Step j:
  //   read the operands of block j + RA (RA steps of LDS latency hidden),
  //   MFMAs of block j (scale products, int8 dots, their conversions; operands read in step j - RA),
  //   fmas of block j - 1, interleaved with those MFMAs.
  // A wave issues its instructions in order, so each MFMA is followed by about as many VALU instructions as cover its
  // time in the matrix pipe (the other wave on the SIMD fills what is left), and the loop is unrolled over the whole
  // LDS ring (NS stages of KB blocks) so every LDS offset is an immediate. Blocks past the
  // end (nb % KB != 0) read a copy of the last block with dw = dx = 0: their products are 0 and fma(f, 0, acc) ==
  // acc (the chain never holds -0), so they add nothing. The results of "block -1" start at zero for the same reason.
  // Operands of step BL of a stage: WT = 64, block BL (ra1 unused); WT = 32, blocks 2 BL (ra0, rb0) and 2 BL + 1
  // (ra1, rb1).
  auto read = [&]<int BUF, int BL>(v4i& ra0, v4i& ra1, v4i& rb0, v4i& rb1, uint16_t& rdw, float& rdx)
      __attribute__((always_inline)) {
    const uint8_t* st = smem + BUF * S::bytes;
    if constexpr (WT == 64) {
      ra0 = *reinterpret_cast<const v4i*>(st + off_a + BL * kRowsT * 32);
      rb0 = *reinterpret_cast<const v4i*>(st + off_b0 + BL * TOK * 32);
      rb1 = *reinterpret_cast<const v4i*>(st + off_b1 + BL * TOK * 32);
      rdw = *reinterpret_cast<const uint16_t*>(st + off_dw + BL * kRowsT * 2);
      rdx = *reinterpret_cast<const float*>(st + off_dx + BL * TOK * 4);
    } else {
      ra0 = *reinterpret_cast<const v4i*>(st + off_a + 2 * BL * kRowsT * 32);
      ra1 = *reinterpret_cast<const v4i*>(st + off_a + (2 * BL + 1) * kRowsT * 32);
      rb0 = *reinterpret_cast<const v4i*>(st + off_b0 + 2 * BL * TOK * 32);
      rb1 = *reinterpret_cast<const v4i*>(st + off_b0 + (2 * BL + 1) * TOK * 32);
      rdw = *reinterpret_cast<const uint16_t*>(st + off_dw + 2 * BL * kRowsT * 2);
      rdx = *reinterpret_cast<const float*>(st + off_dx + 2 * BL * TOK * 4);
    }
  };
  // fmas i0 .. i1 - 1 of one 16-output half. The empty asm keeps them in their region: without it the compiler moves
  // them into a later one, past the MFMAs they are meant to overlap.
  auto fold = [&](v16f& acc, const v16f& f, const v32f& pp, int t, int i0, int i1) __attribute__((always_inline)) {
#pragma unroll
    for (int i = i0; i < i1; ++i) acc[i] = fma_(f[i], pp[16 * t + i], acc[i]);
    asm volatile("" : "+v"(acc));
  };
  // One step: the MFMAs of a block (TOK = 32: two blocks) and the fmas of the previous step, in five regions of one
  // MFMA each; the VALU work of a region covers its MFMA's time in the matrix pipe. I: the step's index in a ring
  // cycle, which picks the register sets: operands op[I % (RA + 1)] (read RA steps earlier), results rs[I % 2], the
  // previous step's results rs[1 - I % 2]; the step first reads the operands of step I + RA (buffer RB, step RBL of
  // that stage) into op[(I + RA) % (RA + 1)]. bl: the step's first block; a lane's scales are zeroed past the matrix (TOK =
  // 32: the lane's block is bl + h).
  struct Ops {
    v4i a0, a1, b0, b1;
    uint16_t dw;  // f16 weight scale as read
    float dx;
  };
  struct Res {
    v16f f0, f1;
    v32f p;
  };
  Ops op[RA + 1];
  Res rs[NS == 2 ? 1 : 2];
  rs[NS == 2 ? 0 : 1].f0 = {};
  rs[NS == 2 ? 0 : 1].f1 = {};
  rs[NS == 2 ? 0 : 1].p = {};
  v16f& acc_b = WT == 64 ? acc1 : acc0;  // the second MFMA's accumulator
  constexpr bool SINGLE = NS == 2;  // one result set: a step folds its own results (three waves per SIMD cover it)
  auto step = [&]<int I, int RB, int RBL>(int bl) __attribute__((always_inline)) {
    const Ops& o = op[I % (RA + 1)];
    Res& r = rs[SINGLE ? 0 : I % 2];
    const Res& pr = rs[SINGLE ? 0 : 1 - I % 2];
    Ops& nx = op[(I + RA) % (RA + 1)];
    const bool live = (WT == 64 ? bl : bl + h) < nb;
    const float dw = live ? half_to_float(o.dw) : 0.0f, dx = live ? o.dx : 0.0f;
    read.template operator()<RB, RBL>(nx.a0, nx.a1, nx.b0, nx.b1, nx.dw, nx.dx);
    if constexpr (SINGLE) {
      r.p = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, dx, zero, 0, 0, 0);
      r.f0 = __builtin_bit_cast(v16f, __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a0, o.b0, magic, 0, 0, 0));
      r.f1 = __builtin_bit_cast(v16f, __builtin_amdgcn_mfma_i32_32x32x32_i8(WT == 64 ? o.a0 : o.a1, o.b1, magic, 0, 0, 0));
      r.f0 = __builtin_amdgcn_mfma_f32_16x16x1f32(-kMagicF, 1.0f, r.f0, 0, 0, 0);
      r.f1 = __builtin_amdgcn_mfma_f32_16x16x1f32(-kMagicF, 1.0f, r.f1, 0, 0, 0);
      fold(acc0, r.f0, r.p, 0, 0, 16);
      fold(acc_b, r.f1, r.p, 1, 0, 16);
      return;
    }
    r.p = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, dx, zero, 0, 0, 0);
    fold(acc0, pr.f0, pr.p, 0, 0, 16);
    __builtin_amdgcn_sched_barrier(0);
    r.f0 = __builtin_bit_cast(v16f, __builtin_amdgcn_mfma_i32_32x32x32_i8(o.a0, o.b0, magic, 0, 0, 0));
    fold(acc_b, pr.f1, pr.p, 1, 0, 8);
    __builtin_amdgcn_sched_barrier(0);
    r.f1 = __builtin_bit_cast(v16f, __builtin_amdgcn_mfma_i32_32x32x32_i8(WT == 64 ? o.a0 : o.a1, o.b1, magic, 0, 0, 0));
    fold(acc_b, pr.f1, pr.p, 1, 8, 16);
    __builtin_amdgcn_sched_barrier(0);
    r.f0 = __builtin_amdgcn_mfma_f32_16x16x1f32(-kMagicF, 1.0f, r.f0, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    r.f1 = __builtin_amdgcn_mfma_f32_16x16x1f32(-kMagicF, 1.0f, r.f1, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // Stage s (steps of blocks KB s ..) from buffer BUF, the BUF-th stage of a ring cycle. Its step k reads the
  // operands of step k + RA, which from step 4 - RA on belong to the next stage, so the next stage is entered before
  // step 4 - RA: it has landed (at most the NS - 2 after it are outstanding) and every wave is done reading this buffer
  // (its last reads were issued in the step before and are waited for here). Stage s + NS then goes into this buffer,
  // a quarter of its copies at the start of each of the four steps that follow: a CU's texture unit takes a 1 KB copy
  // in about 16 cycles, and all of them issued at the entry queued each wave behind the others' (about 80 cycles per
  // copy and wave). All of stage s + NS is issued before the next entry, which counts it as in flight.
  auto enter = [&](int s) __attribute__((always_inline)) {
    if (s + 1 < nstages) {
      __builtin_amdgcn_s_waitcnt(0xC07F);                         // lgkmcnt(0)
      wait_vm_stages<S::loads, NS - 2>(nstages - 2 - s);  // stages s + 2 .. s + NS - 1 may be in flight
      ring_barrier();
    }
  };
  // Quarter P of stage t's copies into buffer BUF.
  auto quarter = [&]<int BUF, int P>(int t) __attribute__((always_inline)) {
    if (t < nstages) copies.template operator()<BUF, P * S::loads / 4, (P + 1) * S::loads / 4>(t);
  };
  auto stage = [&]<int BUF>(int s) __attribute__((always_inline)) {
    constexpr int NBUF = (BUF + 1) % NS, PBUF = (BUF + NS - 1) % NS;
    constexpr int BPS = KB / 4;  // blocks per step
    const int j = s * KB;
    [&]<int... K>(std::integer_sequence<int, K...>) __attribute__((always_inline)) {
      (((K == 4 - RA) ? enter(s) : void(),
        (K >= 4 - RA) ? quarter.template operator()<BUF, (K + RA) % 4>(s + NS)
                      : (s >= 1 ? quarter.template operator()<PBUF, (K + RA) % 4>(s - 1 + NS) : void()),
        live ? step.template operator()<4 * BUF + K, (K + RA < 4 ? BUF : NBUF), (K + RA) % 4>(j + K * BPS) : void()),
       ...);
    }(std::make_integer_sequence<int, 4>{});
  };
  static_assert(RA == 1 || RA == 2, "read-ahead of one or two steps");
  static_assert((4 * NS) % (RA + 1) == 0, "a ring cycle of 4 NS steps keeps the operand sets (mod RA + 1) and result sets (mod 2) in place");

  // Stages 0 .. NS - 2 into buffers 0 .. NS - 2; once stage 0 has landed, stage NS - 1.
  [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
    ((I < nstages ? issue.template operator()<I>(I) : void()), ...);
  }(std::make_integer_sequence<int, NS - 1>{});
  wait_vm_stages<S::loads, NS - 2>(nstages - 1);
  ring_barrier();
  if (NS - 1 < nstages) issue.template operator()<NS - 1>(NS - 1);
  if (live) {
    read.template operator()<0, 0>(op[0].a0, op[0].a1, op[0].b0, op[0].b1, op[0].dw, op[0].dx);
    if constexpr (RA == 2) read.template operator()<0, 1>(op[1].a0, op[1].a1, op[1].b0, op[1].b1, op[1].dw, op[1].dx);
  }
  // Ring cycles, left after the last stage: every stage is four steps, so the register sets are in place at any stage
  // boundary and the last step's results are in rs[1].
  for (int s = 0; s < nstages; s += NS) {
    [&]<int... I>(std::integer_sequence<int, I...>) __attribute__((always_inline)) {
      (void)((s + I < nstages ? (stage.template operator()<I>(s + I), true) : false) && ...);
    }(std::make_integer_sequence<int, NS>{});
  }
  if constexpr (!SINGLE) {
    fold(acc0, rs[1].f0, rs[1].p, 0, 0, 16);
    fold(acc_b, rs[1].f1, rs[1].p, 1, 0, 16);
  }
  // The last stage's loads were waited for (vmcnt(0)) when it was entered; nothing is in flight past the loop.

  // Element i of tile j: row 32 rg + 8 (i / 4) + 4 h + i % 4, token tw + 32 j + li.
  if (32 * rg < 8 * ngroups) {
    float* yr = y + (int64_t)rt * kRowsT + 32 * rg + 4 * h;
#pragma unroll
    for (int j = 0; j < WT / 32; ++j) {
      const int t = t0 + tw + 32 * j + li;
      if (t >= n) continue;
      float* yt = yr + (int64_t)t * ys;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const v16f& av = j ? acc1 : acc0;
        const float v[4] = {av[4 * q], av[4 * q + 1], av[4 * q + 2], av[4 * q + 3]};
        if (vec) {
          float4* p = reinterpret_cast<float4*>(yt + 8 * q);
          float4 o = make_float4(v[0], v[1], v[2], v[3]);
          if (accumulate) {
            const float4 e = *p;
            o = make_float4(e.x + o.x, e.y + o.y, e.z + o.z, e.w + o.w);
          }
          *p = o;
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) yt[8 * q + e] = accumulate ? yt[8 * q + e] + v[e] : v[e];
        }
      }
    }
  }
}

}  // namespace

bool gemm_q8_0_supported(int64_t rows, int64_t cols, int n) { return rows % 32 == 0 && cols % 32 == 0 && n > 8; }

void gemm_q8_0(hipStream_t s, const void* w, int64_t rows, int64_t cols, const BlockQ8* x, int n, float* y, int64_t ys,
               bool accumulate) {
  require(gemm_q8_0_supported(rows, cols, n), "gemm_q8_0: rows must be a multiple of 32, n > 8");
  const int n_rt = (int)((rows + kRowsT - 1) / kRowsT);
  const int vec = (reinterpret_cast<uintptr_t>(y) % 16 == 0 && ys % 4 == 0) ? 1 : 0;
  auto go = [&]<int TOK, int WT, int NS, int RA>() {
    using S = StageLds<TOK, WT>;
    const int n_tt = (n + TOK - 1) / TOK;
    const size_t lds = NS * (size_t)S::bytes;
    static bool attr = false;
    if (!attr) {
      check(hipFuncSetAttribute(reinterpret_cast<const void*>(k_gemm_q8_0<TOK, WT, NS, RA>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds),
            "hipFuncSetAttribute");
      attr = true;
    }
    hipLaunchKernelGGL((k_gemm_q8_0<TOK, WT, NS, RA>), dim3((unsigned)((int64_t)n_rt * n_tt)), dim3(64 * S::NW), lds,
                       s, static_cast<const uint8_t*>(w), rows, cols, x, n, y, ys, accumulate ? 1 : 0, n_rt, n_tt, vec);
  };
  // Forms by grid size, measured on MI355X (bench.py --probe gemm shapes; every form bit-identical): a grid that fits
  // the CUs once at 32-token tiles takes them (4096 x 4096 at 256 tokens: 23.8 us against 29.7 with eight waves); one
  // that fits once at 64-token tiles takes the eight-wave form, two waves per SIMD in one workgroup (4096 x 4096 at 512
  // tokens 40.5 -> 34.0 us, 4096 x 12288 103.1 -> 85.2, 6144 x 4096 at 256 tokens 38.8 -> 32.0, against the
  // four-wave 6-stage ring); grids that fit two four-wave workgroups per CU take those; larger ones three (a two-stage
  // ring and one result set, so that 168 registers hold a wave: config 1's 608 tiles 58.1 -> 53.8 us, gate|up 24576 x
  // 4096 at 512 tokens 187.2 -> 183.2; a grid of one round at two per CU runs slower in it, 6144 x 4096 56.3 -> 56.9).
  const int64_t cus = device_cus();
  if ((int64_t)n_rt * ((n + 31) / 32) <= cus)
    go.template operator()<32, 32, 3, 1>();
  else if ((int64_t)n_rt * ((n + 63) / 64) <= cus)
    go.template operator()<64, 32, 3, 2>();
  else if ((int64_t)n_rt * ((n + 63) / 64) <= 2 * cus)
    go.template operator()<64, 64, 3, 2>();
  else
    go.template operator()<64, 64, 2, 1>();
  check_launch("gemm_q8_0");
}

}  // namespace mk
