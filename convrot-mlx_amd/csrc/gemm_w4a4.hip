// W4A4 GEMM for gfx950 on INT8 MFMA with the scale/bias epilogue fused.
//
// Replaces the reference's MPP int8 x int4 TensorOp kernel plus its separate
// int32 -> output epilogue kernel (/root/reference/src/convrot_mlx/core.py:
// 839-874 and 925-937, launched by mpp_w4a4_int8_matmul :1088-1120 and
// mpp_w4a4_matmul :1061-1085) with the numerics of the eager oracle
// reference_w4a4_matmul (core.py:1155-1171): an exact integer dot, then
// ((float(dot) * xscale[m]) * wscale[n]) + bias[n] in float32, left to right,
// rounded once to the output dtype.  No int32 M x N intermediate touches HBM.
//
// Operands
//  * activations: int8 codes [M, K] row-major (the INT8 prep output), or
//    packed A4 [M, K/2] (low nibble = even feature);
//  * weights: CDNA4 tile layout -- 1 KB blocks of 16 output rows x 128
//    features, block order [K/128][N/16]; lane L = 16q + r of a wave reads
//    the 16 bytes at L*16, i.e. row r, features 32q .. 32q+31, laid out so
//    that (w << 4) & 0xf0f0f0f0 and w & 0xf0f0f0f0 yield the int8 codes x16
//    of features 8c+0..3 and 8c+4..7 of dword c, in natural order.
//
// MFMA mapping: v_mfma_i32_16x16x64_i8 with the weights as the first operand
// (rows = output features n) and the activations as the second (columns =
// tokens m), so each lane's accumulator holds 4 consecutive n of one m and
// the epilogue stores 4 contiguous outputs per lane.  The x16 nibble scaling
// makes every accumulator an exact multiple of 16 (x256 with packed
// activations); |acc| <= 256 * 64 * K < 2^31 for K <= 65536 / 2.
//
// Pipeline: a workgroup of WM x WN waves owns a BM x BN output tile and walks
// K in 128-feature blocks.  Block kb+1 is fetched from HBM/L2 into registers
// while block kb is multiplied out of LDS; the registers are then written to
// the other LDS stage -- two LDS stages, one workgroup barrier per block.
// Workgroups are renumbered so that the tiles one XCD (one L2) runs are
// adjacent in groups of GM tile rows.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "convrot_device.h"
#include "convrot_launch.h"

namespace convrot {
namespace {

constexpr int kXcds = 8;  // MI355X: 8 XCDs, workgroups dispatched round-robin
constexpr int kGroupM = 4;

template <int BM, int BN, int WM, int WN, bool APACK, int ODT>
__global__ __launch_bounds__(WM* WN * 64) void w4a4_gemm_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, GatedResidual gr) {
  constexpr int NT = WM * WN * 64;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int AROW = APACK ? 64 : 128;  // activation bytes per row per 128-feature block
  constexpr int ASTR = AROW + 16;         // padded LDS row stride (conflict-free 16-byte reads)
  constexpr int A_BYTES = BM * ASTR, B_BYTES = BN * 64, STAGE = A_BYTES + B_BYTES;
  constexpr int ACH = BM * AROW / 16;     // 16-byte chunks per block
  constexpr int BCH = BN * 4;             // (BN/16 tiles) x 64 chunks
  constexpr int APT = ACH / NT, BPT = BCH / NT;
  constexpr int SHIFT = APACK ? 8 : 4;    // acc = 2^SHIFT * dot
  static_assert(ACH % NT == 0 && BCH % NT == 0, "tile / thread mismatch");

  __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- XCD-aware tile order
  const int tiles = tiles_m * tiles_n;
  int logical = blockIdx.x;
  const int per_xcd = tiles / kXcds;
  if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
  const int group = logical / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int group_rows = min(kGroupM, tiles_m - first_m);
  const int in_group = logical - group * kGroupM * tiles_n;
  const int m0 = (first_m + in_group % group_rows) * BM;
  const int n0 = (in_group / group_rows) * BN;

  const int64_t arow_bytes = APACK ? (K >> 1) : K;

  uint4 ra[APT], rb[BPT];
  auto gload = [&](int kb) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int c = tid + i * NT;
      const int row = c / (AROW / 16), col = c % (AROW / 16);
      const int gm = m0 + row;
      const int64_t gk = (int64_t)kb * AROW + col * 16;
      ra[i] = (gm < M && gk < arow_bytes) ? *(const uint4*)(act + gm * arow_bytes + gk) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int c = tid + i * NT;
      const int nb = n0 / 16 + c / 64;
      rb[i] = nb < nblocks ? *(const uint4*)(wq + ((int64_t)kb * nblocks + nb) * 1024 + (c % 64) * 16)
                           : make_uint4(0, 0, 0, 0);
    }
  };
  auto sstore = [&](int stage) {
    uint8_t* sA = smem + stage * STAGE;
    uint8_t* sB = sA + A_BYTES;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int c = tid + i * NT;
      *(uint4*)(sA + (c / (AROW / 16)) * ASTR + (c % (AROW / 16)) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) *(uint4*)(sB + (tid + i * NT) * 16) = rb[i];
  };

  i32x4 acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};

  gload(0);
  sstore(0);
  __syncthreads();

  for (int kb = 0; kb < kblocks; ++kb) {
    const bool more = kb + 1 < kblocks;
    if (more) gload(kb + 1);
    const uint8_t* sA = smem + (kb & 1) * STAGE;
    const uint8_t* sB = sA + A_BYTES;

    uint4 bw[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bw[fn] = *(const uint4*)(sB + (wn * FN + fn) * 1024 + lane * 16);

#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      i32x4 bop[FN];
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const uint32_t w0 = ks ? bw[fn].z : bw[fn].x;
        const uint32_t w1 = ks ? bw[fn].w : bw[fn].y;
        uint32_t l0, h0, l1, h1;
        nibbles_x16(w0, l0, h0);
        nibbles_x16(w1, l1, h1);
        bop[fn] = (i32x4){(int)l0, (int)h0, (int)l1, (int)h1};
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * TM + fm * 16 + (lane & 15);
        i32x4 aop;
        if constexpr (!APACK) {
          aop = *(const i32x4*)(sA + row * ASTR + (lane >> 4) * 32 + ks * 16);
        } else {
          // standard packing: byte j = k[2j] | k[2j+1] << 4 -> natural-order int8 x16
          const uint2 p = *(const uint2*)(sA + row * ASTR + (lane >> 4) * 16 + ks * 8);
          const uint32_t e0 = (p.x << 4) & 0xf0f0f0f0u, o0 = p.x & 0xf0f0f0f0u;
          const uint32_t e1 = (p.y << 4) & 0xf0f0f0f0u, o1 = p.y & 0xf0f0f0f0u;
          aop = (i32x4){(int)__builtin_amdgcn_perm(o0, e0, 0x05010400u), (int)__builtin_amdgcn_perm(o0, e0, 0x07030602u),
                        (int)__builtin_amdgcn_perm(o1, e1, 0x05010400u), (int)__builtin_amdgcn_perm(o1, e1, 0x07030602u)};
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fn][fm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bop[fn], aop, acc[fn][fm], 0, 0, 0);
      }
    }
    if (more) sstore((kb + 1) & 1);
    __syncthreads();
  }

  // ---- fused epilogue (core.py:1168-1171): ((dot * xs) * ws) + bias, then round once
  const bool vec_ok = (N & 3) == 0;
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int n = n0 + wn * TN + fn * 16 + 4 * (lane >> 4);
    if (n >= N) continue;
    float wsv[4], bv[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int nn = n + r < N ? n + r : N - 1;
      wsv[r] = wscales[nn];
      bv[r] = bias ? bias[nn] : 0.0f;
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = m0 + wm * TM + fm * 16 + (lane & 15);
      if (m >= M) continue;
      const float xs = xscales[m];
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float v = (float)(acc[fn][fm][r] >> SHIFT);
        v = v * xs;
        v = v * wsv[r];
        v = v + bv[r];
        o[r] = v;
      }
      if (gr.residual) gate_residual4<ODT>(gr, m, n, N, vec_ok, o);
      const int64_t idx = (int64_t)m * N + n;
      if (vec_ok) {
        store_out4<ODT>(out, idx, o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) store_out<ODT>(out, idx + r, o[r]);
      }
    }
  }
}



// Fused epilogue of one wave's TM x TN accumulator tile:
//   out = dtype(((float(acc >> SHIFT) * xs[m]) * ws[n]) + bias[n])   (core.py:1168-1171)
// 16-bit outputs are staged through the wave's LDS region (row stride TN*2+16
// bytes) and written back as 16-byte stores covering whole row segments; the
// MFMA accumulator layout (4 consecutive n of one m per lane) would otherwise
// produce 32-byte write fragments.  float32 outputs store 4 values per lane.
//
// Operands: xs[m], ws[n] and bias[n] come from global memory, or (LDS_OPS)
// from the tile's LDS copies xs[m - m0], ws[n - n0], bias[n - n0] (rows and
// columns past M / N hold zeros there and are never stored).
//
// With gr.residual set, the gated residual follows the rounding of the linear
// (GatedResidual); for 16-bit outputs it is applied in the write-back loop,
// where each lane holds 8 consecutive outputs of one row and loads the
// matching residual and gate elements as 16-byte reads.
//
// `poison` (a stream-K owner whose bounded wait for a partial tile gave up)
// makes every output of the wave's tile NaN instead of a silently wrong value.
// An accumulator element as the float the epilogue scales: int32 sums of
// codes x 2^SHIFT, or (FP6 kernel) the exact float sum of code products.
template <int SHIFT>
__device__ __forceinline__ float acc_value(int v) {
  return (float)(v >> SHIFT);
}
template <int SHIFT>
__device__ __forceinline__ float acc_value(float v) {
  return v;
}

template <int ODT, int TM, int TN, int SHIFT, bool LDS_OPS = false, class V = i32x4, bool PIPE = false>
__device__ __forceinline__ void epilogue(const V (&acc)[TN / 16][TM / 16], uint8_t* region, int lane,
                                         int mw, int nw, int M, int N, const float* __restrict__ xscales,
                                         const float* __restrict__ wscales, const float* __restrict__ bias,
                                         void* __restrict__ out, const GatedResidual& gr, int m0 = 0,
                                         int n0 = 0, bool poison = false) {
  constexpr int FM = TM / 16, FN = TN / 16;
  float xs[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = mw + fm * 16 + (lane & 15);
    if constexpr (LDS_OPS) xs[fm] = xscales[m - m0];
    else xs[fm] = xscales[m < M ? m : M - 1];
    if (poison) xs[fm] = __builtin_nanf("");
  }
  if constexpr (ODT == kF32) {
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int n = nw + fn * 16 + 4 * (lane >> 4);
      if (n >= N) continue;
      float wsv[4], bv[4];
      if constexpr (LDS_OPS) {
        const float4 w4 = *(const float4*)(wscales + (n - n0));
        const float4 b4 = *(const float4*)(bias + (n - n0));
        wsv[0] = w4.x, wsv[1] = w4.y, wsv[2] = w4.z, wsv[3] = w4.w;
        bv[0] = b4.x, bv[1] = b4.y, bv[2] = b4.z, bv[3] = b4.w;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int nn = n + r < N ? n + r : N - 1;
          wsv[r] = wscales[nn];
          bv[r] = bias ? bias[nn] : 0.0f;
        }
      }
      // Residual / gate operands of FB fragments at a time go out before
      // their stores.  The accumulators are still live here: the 128 x 64
      // wave tile (256 x 256 workgroup) has no registers to spare for them.
      constexpr int FB = TM * TN >= 128 * 64 ? 1 : FM;
      Gated4 ops[FB];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if (FB > 1 && gr.residual && fm % FB == 0) {
#pragma unroll
          for (int i = 0; i < FB; ++i) {
            const int m = mw + (fm + i) * 16 + (lane & 15);
            if (m < M) gate_load4<ODT>(gr, m, n, N, vec_ok, ops[i]);
          }
        }
        const int m = mw + fm * 16 + (lane & 15);
        if (m >= M) continue;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = ((acc_value<SHIFT>(acc[fn][fm][r]) * xs[fm]) * wsv[r]) + bv[r];
        if (gr.residual) {
          if constexpr (FB > 1) gate_apply4<ODT>(ops[fm % FB], o);
          else gate_residual4<ODT>(gr, m, n, N, vec_ok, o);
        }
        const int64_t idx = (int64_t)m * N + n;
        if (vec_ok) {
          store_out4<ODT>(out, idx, o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) store_out<ODT>(out, idx + r, o[r]);
        }
      }
    }
  } else {
    constexpr int RS = TN * 2 + 16;  // LDS row stride in bytes
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int nl = fn * 16 + 4 * (lane >> 4);
      float wsv[4], bv[4];
      if constexpr (LDS_OPS) {
        const float4 w4 = *(const float4*)(wscales + (nw + nl - n0));
        const float4 b4 = *(const float4*)(bias + (nw + nl - n0));
        wsv[0] = w4.x, wsv[1] = w4.y, wsv[2] = w4.z, wsv[3] = w4.w;
        bv[0] = b4.x, bv[1] = b4.y, bv[2] = b4.z, bv[3] = b4.w;
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int nn = min(nw + nl + r, N - 1);
          wsv[r] = wscales[nn];
          bv[r] = bias ? bias[nn] : 0.0f;
        }
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = ((acc_value<SHIFT>(acc[fn][fm][r]) * xs[fm]) * wsv[r]) + bv[r];
        const uint2 w = ODT == kBF16 ? make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]))
                                     : make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
        *(uint2*)(region + (fm * 16 + (lane & 15)) * RS + nl * 2) = w;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Write-back: the tile's TM x CPR 16-byte chunks, 64 per wave
    // instruction; chunk c = 64 it + lane is row c / CPR, chunk c % CPR of it.
    constexpr int CPR = TN / 8;                 // 16-byte chunks per row
    constexpr int NIT = (TM * CPR + 63) / 64;   // write-back iterations
    constexpr bool kWhole = (TM * CPR) % 64 == 0;
    auto row_of = [&](int it) { return (it * 64 + lane) / CPR; };
    auto col_of = [&](int it) { return nw + ((it * 64 + lane) % CPR) * 8; };
    auto live = [&](int it) {
      return (kWhole || it * 64 + lane < TM * CPR) && mw + row_of(it) < M && col_of(it) < N;
    };
    auto store_row = [&](int it, uint4 v) {
      const int n = col_of(it);
      uint16_t* dst = (uint16_t*)out + (int64_t)(mw + row_of(it)) * N + n;
      if ((N & 7) == 0 && n + 8 <= N) {
        *(uint4*)dst = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (n + j < N) dst[j] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
      }
    };
    auto staged = [&](int it) {
      return *(const uint4*)(region + row_of(it) * RS + ((it * 64 + lane) % CPR) * 16);
    };
    if (!gr.residual) {
#pragma unroll
      for (int it = 0; it < NIT; ++it)
        if (live(it)) store_row(it, staged(it));
    } else if constexpr (PIPE) {
      // Software-pipelined (kernels with registers to spare after the k-loop):
      // batch b+1's residual and gate loads go out before batch b is applied
      // and stored, so one memory round trip is exposed instead of one per
      // batch.  Batches cover disjoint chunks, so an in-place residual is
      // still read before it is overwritten.
      constexpr int B = NIT < 8 ? NIT : 8, NB = (NIT + B - 1) / B;
      Gated8 ops[2][B];
      auto load_batch = [&](int bi, Gated8(&dst)[B]) {
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const int it = bi * B + i;
          if (it < NIT && live(it)) {
            const int n = col_of(it);
            gate_load8<ODT>(gr, mw + row_of(it), n, N, (N & 7) == 0 && n + 8 <= N, dst[i]);
          }
        }
      };
      load_batch(0, ops[0]);
#pragma unroll
      for (int bi = 0; bi < NB; ++bi) {
        if (bi + 1 < NB) load_batch(bi + 1, ops[(bi + 1) & 1]);
#pragma unroll
        for (int i = 0; i < B; ++i) {
          const int it = bi * B + i;
          if (it < NIT && live(it)) store_row(it, gate_apply8<ODT>(ops[bi & 1][i], staged(it)));
        }
      }
    } else {
      // Residual and gate loads of BATCH rows go out before their stores (a
      // load cannot be moved above a store that may alias it, so one row at a
      // time would wait a memory round trip per row).
      constexpr int BATCH = NIT < 8 ? NIT : 8;
#pragma unroll
      for (int b0 = 0; b0 < NIT; b0 += BATCH) {
        Gated8 ops[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const int it = b0 + i;
          if (it < NIT && live(it)) {
            const int n = col_of(it);
            gate_load8<ODT>(gr, mw + row_of(it), n, N, (N & 7) == 0 && n + 8 <= N, ops[i]);
          }
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const int it = b0 + i;
          if (it < NIT && live(it)) store_row(it, gate_apply8<ODT>(ops[i], staged(it)));
        }
      }
    }
  }
}

// LDS position of a 16-byte chunk of activation row r (128 bytes per row):
// XOR with the row's low three bits and bit 3 keeps 16 consecutive rows of one
// fragment read on distinct banks.
__device__ __forceinline__ int a_swizzle(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// INT8-activation GEMM with direct-to-LDS loads: each 1 KB piece of a
// k-block (8 activation rows x 128 features, or one CDNA4 weight block) is
// fetched by one wave instruction (buffer_load_dwordx4 ... lds) straight into
// an LDS ring of STAGES k-blocks, so no registers stage the data and loads
// run ahead of the MFMAs.  (Three stages suffice: a lone 128x128 workgroup
// runs a k-block in the same ~0.45 us with a 6-deep ring, so it is not
// bound by the bytes in flight.)  Every activation load reads whole 128-byte lines; inside LDS
// the 16-byte chunks of each row are permuted by a_swizzle so that the MFMA
// fragment reads (16 rows x 16 bytes) are bank-conflict free.  Out-of-range
// rows/blocks read as zero through the buffer range check (no branches in the
// loop).
//
// DmaEngine runs any k-range of one BM x BN output tile; the data-parallel
// kernel runs whole tiles with it and the stream-K kernel runs tile pieces.
//
// Fragment pipelines (how LDS reads overlap the MFMAs):
//  kSingle   one register set, read just before the block's MFMAs (the 8-wave
//            256x256 tile: two waves per SIMD cover each other's reads);
//  kPingPong two full sets, block i+1 read during block i's MFMAs;
//  kAgpr     the 4-wave 256x256 tile: one wave per SIMD owns a 128x128 corner
//            whose 64 accumulator fragments fill the 256 AGPRs, and the wave
//            overlaps its own LDS reads with its MFMAs k-step by k-step
//            (body_agpr).  The MFMAs are issued through inline asm: as
//            builtins the compiler routes every MFMA through one AGPR tuple
//            and copies the accumulators around it inside the loop.
enum Pipe : int { kSingle = 0, kPingPong = 1, kAgpr = 2 };

// acc += b . a on the AGPR accumulator c (v_mfma_i32_16x16x64_i8).  The
// "memory" clobber keeps the LDS reads placed between MFMAs where the code
// puts them.  The compiler does not see an MFMA here, so it inserts none of the
// MFMA wait states: the callers pad VALU -> MFMA operand writes
// (hazard_pad) and MFMA -> accumulator reads (mfma_drain) themselves.  Back to
// back accumulation into the same registers needs no padding.
__device__ __forceinline__ void mfma_agpr(i32x4& c, const i32x4& b, const i32x4& a) {
  asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a) : "memory");
}

// Two wait states after the VALU writes of the unpacked weight operands,
// ordered before the MFMAs that read them (the empty asms tie every operand
// to the padding).
template <int FN>
__device__ __forceinline__ void hazard_pad(const i32x4 (&w)[FN]) {
#pragma unroll
  for (int i = 0; i < FN; ++i) asm volatile("" ::"v"(w[i]) : "memory");
  asm volatile("s_nop 1" ::: "memory");
}

// Wait states between the last MFMA and any read of its accumulators (more
// than the 16x16x64 XDL result latency).  Each accumulator is then passed
// through an empty asm that "redefines" it: without that, the compiler is free
// to schedule the epilogue's AGPR reads above the padding, right after the last
// MFMA, since nothing ties them to it.
template <int FN, int FM>
__device__ __forceinline__ void mfma_drain(i32x4 (&acc)[FN][FM]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) asm volatile("" : "+a"(acc[fn][fm]));
}

// The 32 x 32 x 32 form: acc (16 AGPRs, a 32 x 32 int32 block) += b . a.  Lane
// l supplies row l % 32 of each operand and 16 bytes of its k-group l / 32;
// the result's register v of lane l is (n = 8 (v / 4) + 4 (l / 32) + v % 4,
// m = l % 32) of the block.  Hazards as for mfma_agpr (the drain's 24 wait
// states also cover this MFMA's longer result latency).
typedef int i32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ void mfma_agpr32(i32x16& c, const i32x4& b, const i32x4& a) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+a"(c) : "v"(b), "v"(a) : "memory");
}

template <int FN, int FM>
__device__ __forceinline__ void mfma_drain32(i32x16 (&acc)[FN][FM]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) asm volatile("" : "+a"(acc[fn][fm]));
}

// Global slot (0 .. 31) of the second half-block at which DMA piece p of the
// 32 x 32 k-loop is issued: the 12 pieces spread evenly over its 32 MFMAs.
__host__ __device__ constexpr int agpr32_dma_slot(int p) { return p * 8 / 3 + 1; }

template <int BM, int BN, int WM, int WN, int PIPE, int STAGES = 3>
struct DmaEngine {
  static constexpr int kBM = BM, kBN = BN;
  static constexpr int NW = WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int A_FRAGS = (BM / 16) * 2, B_FRAGS = BN / 16;
  static constexpr int LOADS = A_FRAGS + B_FRAGS;
  static constexpr int STAGE_BYTES = LOADS * 1024;
  // Epilogue operands of the tile, loaded into LDS with the first k-blocks:
  // xs[m0 .. m0+BM), ws[n0 .. n0+BN), bias[n0 .. n0+BN), each in whole
  // 256-byte dword DMAs (64 floats).
  static constexpr int XS_DMAS = (BM * 4 + 255) / 256, WS_DMAS = (BN * 4 + 255) / 256;
  static constexpr int EPI_DMAS = XS_DMAS + 2 * WS_DMAS;
  static constexpr int EPI_OFF = STAGES * STAGE_BYTES;
  static constexpr int WS_OFF = EPI_OFF + XS_DMAS * 256, BIAS_OFF = WS_OFF + WS_DMAS * 256;
  static constexpr int EPI_BYTES = EPI_DMAS * 256;
  static constexpr int SMEM_BYTES = EPI_OFF + EPI_BYTES;
  // The persistent kernel keeps two epilogue-operand buffers (the next tile's
  // are fetched while the current tile's are still read).
  static constexpr int SMEM_BYTES_2EPI = EPI_OFF + 2 * EPI_BYTES;

  static constexpr int LPW = LOADS / NW;  // DMA instructions per wave per k-block
  static constexpr int APW = A_FRAGS / NW, BPW = B_FRAGS / NW;  // of which activation / weight
  static constexpr int SHIFT = 4;         // weights unpacked x16: acc = 16 * dot
  static constexpr int STAGING = TM * (TN * 2 + 16);  // epilogue LDS bytes per wave
  static_assert(LOADS % NW == 0, "fragment loads must split evenly over waves");
  static_assert(A_FRAGS % NW == 0 && B_FRAGS % NW == 0, "each wave loads APW + BPW pieces");
  static_assert(NW * STAGING <= EPI_OFF, "epilogue staging exceeds the ring");
  static_assert(SMEM_BYTES <= 160 * 1024, "LDS of one CU");
  static_assert(STAGES >= 3 && (STAGES - 1) * LPW <= 63, "ring depth: vmcnt counts at most 63 DMAs");

  // Fragments of one k-block held in registers: packed weights (both k-steps)
  // and int8 activations for k-steps 0 and 1.
  struct Frags {
    uint4 b[FN];
    i32x4 a[2][FM];
  };

  uint8_t* smem;
  uint32_t smem_addr;
  int lane, wave, wm, wn;
  int epi_buf = 0;  // epilogue-operand buffer in use (0 or 1; 1 only in the persistent kernel)
  // This wave's loads: activation pieces j = wave APW + i (rows 8j .. 8j+7)
  // and weight blocks j = wave BPW + i.  Per-lane byte offsets: va[i & 1]
  // for activations (the row swizzle flips with the parity of j; set_tile
  // swaps the pair where APW and wave are odd, so that i's parity selects
  // it), vb for weights; the rest of each offset is
  // wave-uniform and added at issue time (it changes with k, so the sums are
  // never hoisted into registers).
  i32x4_sgpr ra, rw;
  uint32_t va[2], vb;
  uint32_t a_kstride, w_kstride, krow;

  __device__ __forceinline__ explicit DmaEngine(uint8_t* s) : smem(s) {
    smem_addr = (uint32_t)(uintptr_t)s;
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave / WN;
    wn = wave % WN;
  }

  __device__ __forceinline__ uint8_t* staging() const { return smem + wave * STAGING; }
  __device__ __forceinline__ const float* epi_xs() const {
    return (const float*)(smem + EPI_OFF + epi_buf * EPI_BYTES);
  }
  __device__ __forceinline__ const float* epi_ws() const {
    return (const float*)(smem + WS_OFF + epi_buf * EPI_BYTES);
  }
  __device__ __forceinline__ const float* epi_bias() const {
    return (const float*)(smem + BIAS_OFF + epi_buf * EPI_BYTES);
  }

  // Load the tile's epilogue operands into LDS: EPI_DMAS dword DMAs of 256
  // bytes, DMA d by wave d % NW.  Entries past M or N, and all of a missing
  // bias, read as zero.  Issued before the run's prologue: vmcnt retires in
  // issue order, so the run's first DMA wait also retires these, and the
  // barrier after the run publishes them to every wave.  The area must not be
  // read by a previous epilogue when they are issued.
  __device__ __forceinline__ void issue_epi(const float* xscales, const float* wscales, const float* bias, int M,
                                            int N, int m0, int n0) {
    for (int d = wave; d < EPI_DMAS; d += NW) {  // array arr, 256-byte piece q of it
      const int arr = d < XS_DMAS ? 0 : d < XS_DMAS + WS_DMAS ? 1 : 2;
      const int q = d - (arr == 0 ? 0 : arr == 1 ? XS_DMAS : XS_DMAS + WS_DMAS);
      const int off = (arr == 0 ? EPI_OFF : arr == 1 ? WS_OFF : BIAS_OFF) + epi_buf * EPI_BYTES;
      const float* base = arr == 0 ? xscales + m0 : arr == 1 ? wscales + n0 : (bias ? bias + n0 : wscales);
      const int count = arr == 0 ? M - m0 : (arr == 1 || bias) ? N - n0 : 0;
      const i32x4_sgpr r = buffer_rsrc(base, (uint32_t)count * 4u);
      dma4(r, (uint32_t)(q * 256 + lane * 4), smem_addr + (uint32_t)(off + q * 256));
    }
  }

  // Point the loads at the output tile whose top-left corner is (m0, n0).
  __device__ __forceinline__ void set_tile(const int8_t* act, const uint8_t* wq, int M, int K, int nblocks,
                                           int kblocks, int m0, int n0) {
    const int rows_valid = min(BM, M - m0);
    ra = buffer_rsrc(act + (int64_t)m0 * K, (uint32_t)rows_valid * (uint32_t)K);
    const uint8_t* wbase = wq + (int64_t)(n0 / 16) * 1024;
    const uint32_t wbytes = (uint32_t)(((int64_t)kblocks * nblocks - n0 / 16) * 1024);
    rw = buffer_rsrc(wbase, wbytes);
    // Activation piece j: lane L reads row 8j + (L >> 3), 16-byte chunk
    // (L & 7) ^ swz(row) of the row's 128 bytes (whole cache lines), where
    // swz(row) = (L >> 3) ^ (j & 1).  The row term 8 j K stays in the
    // per-lane offset so rows at or beyond M fail the buffer range check.
    const int rl = lane >> 3, c = lane & 7;
    const int flip = (APW & 1) ? (wave & 1) : 0;  // parity of j = wave APW + i, beyond i's
    va[0] = (uint32_t)(rl * K + 16 * (c ^ rl ^ flip));
    va[1] = (uint32_t)(rl * K + 16 * (c ^ rl ^ flip ^ 1));
    vb = (uint32_t)lane * 16u;
    krow = 8u * (uint32_t)K;
    a_kstride = 128u;
    w_kstride = (uint32_t)nblocks * 1024u;
  }

  __device__ __forceinline__ void issue(int kb, int stage) {
    const uint32_t base = smem_addr + (uint32_t)(stage * STAGE_BYTES);
    // The scalar parts go through an empty asm so the compiler cannot split
    // off their loop-invariant share and keep one register per load.
#pragma unroll
    for (int i = 0; i < APW; ++i) {
      const uint32_t j = (uint32_t)(wave * APW + i);
      uint32_t so = j * krow + (uint32_t)kb * a_kstride;
      asm volatile("" : "+s"(so));
      dma16(ra, va[i & 1] + so, base + j * 1024u);
    }
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const uint32_t j = (uint32_t)(wave * BPW + i);
      uint32_t so = j * 1024u + (uint32_t)kb * w_kstride;
      asm volatile("" : "+s"(so));
      dma16(rw, vb + so, base + (uint32_t)(A_FRAGS + j) * 1024u);
    }
  }

  __device__ __forceinline__ void read_frags(int stage, Frags& f) const {
    const uint8_t* st = smem + stage * STAGE_BYTES;
    const uint8_t* sb = st + (A_FRAGS + wn * FN) * 1024 + lane * 16;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) f.b[fn] = *(const uint4*)(sb + fn * 1024);
    // Row (wm FM + fm) 16 + (lane & 15) holds features 32q + 16ks .. +16 in
    // chunk (2q + ks) ^ swz(row); swz depends on row & 15 = lane & 15 only, so
    // one address per k-step serves every fm (fm adds 2 KB, an immediate).
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int r = lane & 15;
      const uint8_t* sa = st + (wm * FM * 16 + r) * 128 + (((2 * (lane >> 4) + ks) ^ a_swizzle(r)) * 16);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) f.a[ks][fm] = *(const i32x4*)(sa + fm * 2048);
    }
  }

  __device__ __forceinline__ static void mma(const Frags& f, i32x4 (&acc)[FN][FM]) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      i32x4 bop[FN];
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const uint32_t w0 = ks ? f.b[fn].z : f.b[fn].x;
        const uint32_t w1 = ks ? f.b[fn].w : f.b[fn].y;
        uint32_t l0, h0, l1, h1;
        nibbles_x16(w0, l0, h0);
        nibbles_x16(w1, l1, h1);
        bop[fn] = (i32x4){(int)l0, (int)h0, (int)l1, (int)h1};
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fn][fm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bop[fn], f.a[ks][fm], acc[fn][fm], 0, 0, 0);
    }
  }

  // acc += the products over k-blocks kb0 .. kb0+n-1 (n >= 1).  Every DMA has
  // retired on return; the caller puts a barrier between this and any reuse
  // of the ring (epilogue staging or the next run).
  __device__ __forceinline__ void run(int kb0, int n, i32x4 (&acc)[FN][FM]) {
    prologue(kb0, n);
    body_any(kb0, n, acc, nullptr, 0);
  }

  // The pipeline of this engine's PIPE for k-blocks kb0 .. kb0+n-1, after
  // prologue(kb0, n).  With `flag` set, lane 0 of each wave stores `tag` there
  // once its first DMA wait has retired everything the wave issued before the
  // prologue (a stream-K partial tile's stores).
  __device__ __forceinline__ void body_any(int kb0, int n, i32x4 (&acc)[FN][FM], int* flag, int tag) {
    if constexpr (PIPE == kAgpr) body_agpr(kb0, n, acc, flag, tag);
    else body(kb0, n, acc, flag, tag);
  }

  // ---- kAgpr: the 4-wave tiles, one wave per SIMD, FN x FM accumulator
  //      fragments per wave in the AGPRs (256x256: 8 x 8; 288x192: 6 x 9)
  //
  // Per k-block i (two 64-feature k-steps):
  //   k-step 0: FM*FN MFMAs on (w0, a0); between them the wave reads a1 (its
  //             k-step-1 activation fragments) and unpacks w1 from bp;
  //   middle:   the wave's DMAs of block i+1 have landed and its a1 reads are
  //             done; a barrier publishes block i+1 to every wave and frees
  //             block i's ring stage, which the DMA of block i+STAGES refills;
  //   k-step 1: FM*FN MFMAs on (w1, a1); between them the wave reads block
  //             i+1's packed weights bp and k-step-0 fragments a0, and unpacks
  //             w0.
  // So the MFMA pipe never waits for a whole block's reads, and the only
  // workgroup barrier of a block sits between its two k-steps.
  __device__ __forceinline__ void read_bp(int stage, uint4 (&bp)[FN]) const {
    const uint8_t* sb = smem + stage * STAGE_BYTES + (A_FRAGS + wn * FN) * 1024 + lane * 16;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) bp[fn] = *(const uint4*)(sb + fn * 1024);
  }
  __device__ __forceinline__ const uint8_t* a_base(int stage, int ks) const {
    const int r = lane & 15;
    return smem + stage * STAGE_BYTES + (wm * FM * 16 + r) * 128 + (((2 * (lane >> 4) + ks) ^ a_swizzle(r)) * 16);
  }
  __device__ __forceinline__ static void unpack(const uint4& b, int ks, i32x4& w) {
    uint32_t l0, h0, l1, h1;
    nibbles_x16(ks ? b.z : b.x, l0, h0);
    nibbles_x16(ks ? b.w : b.y, l1, h1);
    w = (i32x4){(int)l0, (int)h0, (int)l1, (int)h1};
  }

  // One DMA piece of k-block kb into ring stage `stage`: pieces 0 .. APW-1
  // are this wave's activation pieces, APW .. LPW-1 its weight blocks (the
  // order of issue()).
  __device__ __forceinline__ void issue_piece(int kb, int stage, int idx) {
    const uint32_t base = smem_addr + (uint32_t)(stage * STAGE_BYTES);
    if (idx < APW) {
      const uint32_t j = (uint32_t)(wave * APW + idx);
      uint32_t so = j * krow + (uint32_t)kb * a_kstride;
      asm volatile("" : "+s"(so));
      dma16(ra, va[idx & 1] + so, base + j * 1024u);
    } else {
      const uint32_t j = (uint32_t)(wave * BPW + idx - APW);
      uint32_t so = j * 1024u + (uint32_t)kb * w_kstride;
      asm volatile("" : "+s"(so));
      dma16(rw, vb + so, base + (uint32_t)(A_FRAGS + j) * 1024u);
    }
  }

  // Half of the unpack of one k-step's weight operand (two of its four
  // dwords, from packed dword `src`), placed by the two empty asms exactly where
  // the call sits between two MFMAs: the first makes the source look freshly
  // produced there, the second consumes the results there.
  __device__ __forceinline__ static void unpack_half(uint32_t src, uint32_t& lo, uint32_t& hi) {
    asm volatile("" : "+v"(src));
    nibbles_x16(src, lo, hi);
    asm volatile("" ::"v"(lo), "v"(hi));
  }

  // Filler work between the MFMAs of a k-step: with one wave per SIMD the
  // wave issues about one instruction per four cycles, so LDS reads, weight
  // unpacks and DMA issues placed one or two at a time between MFMAs (16
  // cycles each) run in the MFMA's shadow, where a burst of them would leave
  // the MFMA pipe idle.  Slot t follows MFMA t = FN * fm + fn.
  static constexpr int kSlots = FM * FN;

  // k-step 0 of the block in ring stage st: MFMAs on (w0, a0); read of a1[i]
  // after slot 4i + 1 and half j of the unpack of w1 after slot 4j + 3.
  __device__ __forceinline__ void agpr_kstep0(int st, const uint4 (&bp)[FN], const i32x4 (&a0)[FM],
                                              i32x4 (&a1)[FM], const i32x4 (&w0)[FN], i32x4 (&w1)[FN],
                                              i32x4 (&acc)[FN][FM]) const {
    hazard_pad(w0);
    const uint8_t* sa = a_base(st, 1);
    uint32_t u[FN][4];
#pragma unroll
    for (int t = 0; t < kSlots; ++t) {
      const int fm = t / FN, fn = t % FN;
      mfma_agpr(acc[fn][fm], w0[fn], a0[fm]);
      if (t % 4 == 1 && t / 4 < FM) a1[t / 4] = *(const i32x4*)(sa + (t / 4) * 2048);
      if (t % 4 == 3 && t / 4 < 2 * FN) {
        const int j = t / 8, h = (t / 4) % 2;
        unpack_half(h ? bp[j].w : bp[j].z, u[j][2 * h], u[j][2 * h + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) w1[j] = (i32x4){(int)u[j][0], (int)u[j][1], (int)u[j][2], (int)u[j][3]};
  }

  // k-step 1: MFMAs on (w1, a1); from ring stage nst, reads of the next
  // block's bp[i] after slot 2i and a0[i] after slot 2 FN + 2i; the LPW DMA
  // pieces of k-block dma_kb into stage st after slots 1, 5, 9, ..; half j of
  // the unpack of the next w0 after slot 2 (FN + FM) + 1 + 2j.
  __device__ __forceinline__ void agpr_kstep1(int st, int nst, int dma_kb, uint4 (&bp)[FN], i32x4 (&a0)[FM],
                                              const i32x4 (&a1)[FM], i32x4 (&w0)[FN], const i32x4 (&w1)[FN],
                                              i32x4 (&acc)[FN][FM]) {
    constexpr int U0 = 2 * (FN + FM) + 1;
    hazard_pad(w1);
    const uint8_t* sa = a_base(nst, 0);
    const uint8_t* sb = smem + nst * STAGE_BYTES + (A_FRAGS + wn * FN) * 1024 + lane * 16;
    uint32_t u[FN][4];
#pragma unroll
    for (int t = 0; t < kSlots; ++t) {
      const int fm = t / FN, fn = t % FN;
      mfma_agpr(acc[fn][fm], w1[fn], a1[fm]);
      if (t % 2 == 0 && t < 2 * FN) bp[t / 2] = *(const uint4*)(sb + (t / 2) * 1024);
      if (t % 2 == 0 && t >= 2 * FN && t < 2 * (FN + FM))
        a0[(t - 2 * FN) / 2] = *(const i32x4*)(sa + ((t - 2 * FN) / 2) * 2048);
      if (t % 4 == 1 && t / 4 < LPW) issue_piece(dma_kb, st, t / 4);
      if (t >= U0 && (t - U0) % 2 == 0 && (t - U0) / 2 < 2 * FN) {
        const int k = (t - U0) / 2, j = k / 2, h = k % 2;
        unpack_half(h ? bp[j].y : bp[j].x, u[j][2 * h], u[j][2 * h + 1]);
      }
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) w0[j] = (i32x4){(int)u[j][0], (int)u[j][1], (int)u[j][2], (int)u[j][3]};
  }

  // The k-loop runs one branch-free body per block, so the accumulators keep
  // one live range (and one set of AGPRs): the last block still reads a "next"
  // block from a ring stage nothing reads afterwards, and DMAs past the run's
  // last k-block re-fetch that last block (in range) into stages no later
  // block uses.  Two DMA groups are therefore in flight at every middle wait.
  __device__ __forceinline__ void body_agpr(int kb0, int n, i32x4 (&acc)[FN][FM], int* flag, int tag) {
    static_assert(NW == 4 && STAGES == 3, "kAgpr: 4 waves, 3 stages");
    static_assert(4 * (FM > 2 * FN ? FM : 2 * FN) <= kSlots, "k-step 0 fillers: one per four slots");
    static_assert(2 * (FN + FM) + 2 * (2 * FN) - 1 <= kSlots && 4 * LPW - 3 <= kSlots,
                  "k-step 1 fillers: reads, DMA pieces and unpacks");
    uint4 bp[FN];
    i32x4 a0[FM], a1[FM], w0[FN], w1[FN];
    wait_vmcnt<2 * LPW>();  // block 0 (and the epilogue operands) landed
    if (flag && lane == 0) __hip_atomic_store(flag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_barrier();
    read_bp(0, bp);
    {
      const uint8_t* sa = a_base(0, 0);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) a0[fm] = *(const i32x4*)(sa + fm * 2048);
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) unpack(bp[fn], 0, w0[fn]);
    const int last_kb = kb0 + n - 1;
    int st = 0;
    for (int i = 0; i < n; ++i) {
      const int nst = st + 1 == STAGES ? 0 : st + 1;
      agpr_kstep0(st, bp, a0, a1, w0, w1, acc);
      // middle: the wave's DMAs of block i+1 and its a1 reads are done; the
      // barrier publishes block i+1 to every wave and frees stage st
      wait_vmcnt<LPW>();
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      agpr_kstep1(st, nst, min(kb0 + i + STAGES, last_kb), bp, a0, a1, w0, w1, acc);
      st = nst;
    }
    mfma_drain(acc);
    wait_vmcnt<0>();  // the DMAs past the last block have landed before the ring is reused
  }

  // ---- kAgpr on v_mfma_i32_32x32x32_i8: the wave's TM x TN corner as
  //      FN32 x FM32 blocks of 32 x 32, four 32-feature k-steps per k-block.
  //
  // Lane (g = lane / 32, r = lane % 32) feeds row r of a block and, in k-step
  // s, the 16 features of 16-byte chunk c = 4 g + s of the k-block: activation
  // chunk c of row r; weight row r (CDNA4 weight block 2 f + r / 16, row r % 16)
  // holds chunks 2 q and 2 q + 1 in the 16 bytes of layout lane 16 q + r % 16,
  // so the lane reads q = 2 g (chunks 4 g, 4 g + 1) and q = 2 g + 1 (4 g + 2,
  // 4 g + 3).  Both operands pair chunk c byte for byte as the 16 x 16 x 64
  // path does, so the integer dot products are the same.
  //
  // Per k-block: k-steps 0 and 1 read the block's activation chunks for
  // k-steps 1 .. 3; a barrier publishes block i+1 and frees the block's ring
  // stage; k-steps 2 and 3 read block i+1's packed weights and k-step-0
  // activations and issue the 12 DMA pieces of block i+STAGES.
  static constexpr int FN32 = TN / 32, FM32 = TM / 32, NS32 = FN32 * FM32;

  __device__ __forceinline__ const uint8_t* a_base32(int stage, int s) const {
    const int r = lane & 31;
    return smem + stage * STAGE_BYTES + (wm * TM + r) * 128 + (((4 * (lane >> 5) + s) ^ a_swizzle(r)) * 16);
  }
  // Packed weights of block f, half q - 2 g of the lane: at + f * 2048 + i * 256.
  __device__ __forceinline__ const uint8_t* b_base32(int stage) const {
    return smem + stage * STAGE_BYTES + (A_FRAGS + wn * FN + ((lane >> 4) & 1)) * 1024 +
           (32 * (lane >> 5) + (lane & 15)) * 16;
  }
  __device__ __forceinline__ void read_bq32(int stage, uint4 (&bq)[FN32][2]) const {
    const uint8_t* sb = b_base32(stage);
#pragma unroll
    for (int f = 0; f < FN32; ++f)
#pragma unroll
      for (int i = 0; i < 2; ++i) bq[f][i] = *(const uint4*)(sb + f * 2048 + i * 256);
  }

  // k-step S of the block in ring stage st: MFMAs on (w[S & 1], a[S]); the
  // fillers between them prepare the following k-steps (see above).
  template <int S>
  __device__ __forceinline__ void agpr32_kstep(int st, int nst, int dma_kb, uint4 (&bq)[FN32][2],
                                               i32x4 (&a)[4][FM32], i32x4 (&w)[2][FN32],
                                               i32x16 (&acc)[FN32][FM32]) {
    hazard_pad(w[S & 1]);
    uint32_t u[FN32][4];
    // source of the next k-step's weights: this block's bq, or (S == 3) the next block's
    constexpr int NB = S == 3 ? 0 : (S + 1) >> 1, NH = (S + 1) & 1;
    const uint8_t* sa1 = a_base32(S < 2 ? st : nst, S == 0 ? 1 : S == 1 ? 3 : 0);
    const uint8_t* sa2 = a_base32(st, 2);
    const uint8_t* sb = b_base32(nst);
#pragma unroll
    for (int t = 0; t < NS32; ++t) {
      const int fm = t / FN32, fn = t % FN32;
      mfma_agpr32(acc[fn][fm], w[S & 1][fn], a[S][fm]);
      // activation chunks: S 0 -> a[1] at slots 1, 3, .. and a[2] after them;
      // S 1 -> a[3]; S 3 -> next block's a[0] (ring stage nst)
      if (S != 2 && t % 2 == 1 && t / 2 < FM32) {
        if constexpr (S == 0) a[1][t / 2] = *(const i32x4*)(sa1 + (t / 2) * 4096);
        if constexpr (S == 1) a[3][t / 2] = *(const i32x4*)(sa1 + (t / 2) * 4096);
        if constexpr (S == 3) a[0][t / 2] = *(const i32x4*)(sa1 + (t / 2) * 4096);
      }
      if (S == 0 && t % 2 == 1 && t / 2 >= FM32 && t / 2 < 2 * FM32)
        a[2][t / 2 - FM32] = *(const i32x4*)(sa2 + (t / 2 - FM32) * 4096);
      // S 2: the next block's packed weights (ring stage nst) after this
      // block's last unpack (slots 0 .. 2 FN32 - 1 below)
      if (S == 2 && t >= 2 * FN32 && t < 4 * FN32) {
        const int k = t - 2 * FN32;
        bq[k / 2][k % 2] = *(const uint4*)(sb + (k / 2) * 2048 + (k % 2) * 256);
      }
      // DMA pieces of block dma_kb into the freed stage st
      if (S >= 2) {
#pragma unroll
        for (int p = 0; p < LPW; ++p)
          if (agpr32_dma_slot(p) == (S - 2) * NS32 + t) issue_piece(dma_kb, st, p);
      }
      // the next k-step's weight operand, half k of 2 FN32: S 0..2 at slots
      // 0 .. 2 FN32 - 1 (S 0, 1 on even slots), S 3 once its bq has landed
      {
        int k = -1;
        if (S == 0 || S == 1) k = t % 2 == 0 ? t / 2 : -1;
        if (S == 2) k = t;
        if (S == 3) k = t - (NS32 - 2 * FN32);
        if (k >= 0 && k < 2 * FN32) {
          const int j = k / 2, h = k % 2;
          const uint4& b = bq[j][NB];
          unpack_half(NH ? (h ? b.w : b.z) : (h ? b.y : b.x), u[j][2 * h], u[j][2 * h + 1]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < FN32; ++j)
      w[(S + 1) & 1][j] = (i32x4){(int)u[j][0], (int)u[j][1], (int)u[j][2], (int)u[j][3]};
  }

  __device__ __forceinline__ void body_agpr32(int kb0, int n, i32x16 (&acc)[FN32][FM32]) {
    static_assert(NW == 4 && STAGES == 3 && TM % 32 == 0 && TN % 32 == 0, "kAgpr 32x32: 4 waves, 3 stages");
    static_assert(NS32 == 16 && FN32 == 4 && FM32 == 4, "filler schedule written for 4 x 4 blocks per wave");
    static_assert(LPW == 12 && agpr32_dma_slot(LPW - 1) < 2 * NS32, "DMA pieces fit the second half-block");
    uint4 bq[FN32][2];
    i32x4 a[4][FM32], w[2][FN32];
    wait_vmcnt<2 * LPW>();  // block 0 (and the epilogue operands) landed
    __builtin_amdgcn_s_barrier();
    read_bq32(0, bq);
    {
      const uint8_t* sa = a_base32(0, 0);
#pragma unroll
      for (int fm = 0; fm < FM32; ++fm) a[0][fm] = *(const i32x4*)(sa + fm * 4096);
    }
#pragma unroll
    for (int f = 0; f < FN32; ++f) unpack(bq[f][0], 0, w[0][f]);
    const int last_kb = kb0 + n - 1;
    int st = 0;
    for (int i = 0; i < n; ++i) {
      const int nst = st + 1 == STAGES ? 0 : st + 1;
      const int dma_kb = min(kb0 + i + STAGES, last_kb);
      agpr32_kstep<0>(st, nst, dma_kb, bq, a, w, acc);
      agpr32_kstep<1>(st, nst, dma_kb, bq, a, w, acc);
      // middle: block i+1 landed and this block's activation reads are done;
      // the barrier publishes block i+1 and frees stage st
      wait_vmcnt<LPW>();
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      agpr32_kstep<2>(st, nst, dma_kb, bq, a, w, acc);
      agpr32_kstep<3>(st, nst, dma_kb, bq, a, w, acc);
      st = nst;
    }
    mfma_drain32(acc);
    wait_vmcnt<0>();  // the DMAs past the last block have landed before the ring is reused
  }

  // Wait until at most `ahead` k-blocks of this wave's DMAs (LPW each) are in
  // flight (`ahead` <= J; wave-uniform, so the branches are scalar).
  template <int J>
  __device__ __forceinline__ static void wait_blocks(int ahead) {
    if constexpr (J <= 0) {
      wait_vmcnt<0>();
    } else {
      if (ahead >= J) wait_vmcnt<J * LPW>();
      else wait_blocks<J - 1>(ahead);
    }
  }

  // First DMAs of a run: k-blocks kb0 .. kb0+STAGES-1 (kPingPong) or
  // kb0 .. kb0+STAGES-2 (kSingle) into stages 0, 1, ...  The ring must be free
  // (barrier after its last reads).
  __device__ __forceinline__ void prologue(int kb0, int n) {
    constexpr int AHEAD = PIPE == kSingle ? STAGES - 1 : STAGES;
#pragma unroll
    for (int s = 0; s < AHEAD; ++s) {
      if constexpr (PIPE == kAgpr) issue(kb0 + min(s, n - 1), s);  // always STAGES groups (body_agpr)
      else if (s < n) issue(kb0 + s, s);
    }
  }

  // The rest of a run after prologue(kb0, n).  The prologue's DMAs must be the
  // newest vector-memory operations of the wave.  vmcnt retires in issue
  // order, so the first wait also retires everything the wave issued before
  // the prologue; if `flag` is set, lane 0 raises it right after that wait.
  __device__ __forceinline__ void body(int kb0, int n, i32x4 (&acc)[FN][FM], int* flag, int tag) {
    auto raise = [&]() {
      if (flag && lane == 0) __hip_atomic_store(flag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    Frags f0;
    if constexpr (PIPE == kPingPong) {
      // DMA STAGES blocks ahead; block i+1's fragments are read into the spare
      // register set while block i's MFMAs run.  The barrier of step i
      // publishes DMA(i+1) and retires every wave's reads of stage i % STAGES
      // (issued in step i-1), which DMA(i+STAGES) then refills.
      Frags f1;
      wait_blocks<STAGES - 1>(min(n, STAGES) - 1);
      raise();
      __syncthreads();
      read_frags(0, f0);
      auto step = [&](int i, Frags& cur, Frags& nxt) {
        // in flight: blocks i+1 .. min(n, i+STAGES)-1; block i+1 must land
        wait_blocks<STAGES - 2>(min(n - i - 2, STAGES - 2));
        __syncthreads();
        if (i + STAGES < n) issue(kb0 + i + STAGES, i % STAGES);
        if (i + 1 < n) read_frags((i + 1) % STAGES, nxt);
        mma(cur, acc);
      };
      int i = 0;
      for (; i + 1 < n; i += 2) {
        step(i, f0, f1);
        step(i + 1, f1, f0);
      }
      if (i < n) step(i, f0, f1);
    } else {
      // One register set: DMA STAGES-1 blocks ahead.  The barrier of
      // iteration i publishes DMA(i) and retires every wave's reads of stage
      // (i-1) % STAGES, which DMA(i+STAGES-1) then refills.
      for (int i = 0; i < n; ++i) {
        wait_blocks<STAGES - 2>(min(n - i - 1, STAGES - 2));
        if (i == 0) raise();
        __syncthreads();
        if (i + STAGES - 1 < n) issue(kb0 + i + STAGES - 1, (i + STAGES - 1) % STAGES);
        read_frags(i % STAGES, f0);
        // Issue all of the block's fragment reads before its MFMAs; left to
        // itself the compiler reads two fragments at a time just before use
        // and the MFMA pipe waits out each LDS round trip.
        __builtin_amdgcn_sched_barrier(0);
        mma(f0, acc);
      }
    }
  }
};

// Top-left corner of logical tile `t`: tiles are walked kGroupM tile rows at
// a time, N-major inside a group, so consecutive tiles share activation rows.
__device__ __forceinline__ void tile_origin(int t, int tiles_m, int tiles_n, int bm, int bn, int& m0, int& n0) {
  const int group = t / (kGroupM * tiles_n);
  const int first_m = group * kGroupM;
  const int group_rows = min(kGroupM, tiles_m - first_m);
  const int in_group = t - group * kGroupM * tiles_n;
  m0 = (first_m + in_group % group_rows) * bm;
  n0 = (in_group / group_rows) * bn;
}

// One workgroup per output tile.  Workgroups are renumbered so that the
// tiles one XCD (one L2) runs are adjacent in the grouped tile order.
template <int BM, int BN, int WM, int WN, int PIPE, int STAGES, int ODT>
__global__ __launch_bounds__(WM* WN * 64) void w4a4_gemm_dma_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, GatedResidual gr) {
  using E = DmaEngine<BM, BN, WM, WN, PIPE, STAGES>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  E e(smem);

  const int tiles = tiles_m * tiles_n;
  int logical = blockIdx.x;
  const int per_xcd = tiles / kXcds;
  if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
  int m0, n0;
  tile_origin(logical, tiles_m, tiles_n, BM, BN, m0, n0);

  e.set_tile(act, wq, M, K, nblocks, kblocks, m0, n0);
  e.issue_epi(xscales, wscales, bias, M, N, m0, n0);
  i32x4 acc[E::FN][E::FM];
#pragma unroll
  for (int a = 0; a < E::FN; ++a)
#pragma unroll
    for (int b = 0; b < E::FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};
  e.run(0, kblocks, acc);
  __syncthreads();  // all waves done with the LDS ring before it is reused for output staging
  epilogue<ODT, E::TM, E::TN, E::SHIFT, true>(acc, e.staging(), e.lane, m0 + e.wm * E::TM, n0 + e.wn * E::TN, M,
                                              N, e.epi_xs(), e.epi_ws(), e.epi_bias(), out, gr, m0, n0);
}

// The kAgpr 4-wave tiles (256x256, 288x192), one workgroup per output tile:
// one wave per SIMD may use all 512 registers (256 VGPRs + the 256 AGPRs of
// the accumulator).
template <int BM, int BN, int STAGES, int ODT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void w4a4_gemm_agpr_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, GatedResidual gr) {
  using E = DmaEngine<BM, BN, 2, 2, kAgpr, STAGES>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  E e(smem);

  const int tiles = tiles_m * tiles_n;
  int logical = blockIdx.x;
  const int per_xcd = tiles / kXcds;
  if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
  int m0, n0;
  tile_origin(logical, tiles_m, tiles_n, BM, BN, m0, n0);

  e.set_tile(act, wq, M, K, nblocks, kblocks, m0, n0);
  e.issue_epi(xscales, wscales, bias, M, N, m0, n0);
  i32x4 acc[E::FN][E::FM];
#pragma unroll
  for (int a = 0; a < E::FN; ++a)
#pragma unroll
    for (int b = 0; b < E::FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};
  e.run(0, kblocks, acc);
  __syncthreads();  // all waves done with the LDS ring before it is reused for output staging
  epilogue<ODT, E::TM, E::TN, E::SHIFT, true, i32x4, true>(acc, e.staging(), e.lane, m0 + e.wm * E::TM,
                                                           n0 + e.wn * E::TN, M, N, e.epi_xs(), e.epi_ws(),
                                                           e.epi_bias(), out, gr, m0, n0);
}

// One pass of the 16-bit epilogue of the persistent 4-wave kernel: fragment
// rows FM0 .. FM1-1 of the wave's TM x TN tile, ((float(acc) * xs) * ws) + bias
// as in `epilogue`, staged through the wave's LDS region and written as 16-byte
// buffer stores; a chunk outside the M x N output gets an offset past the
// buffer's range, which the hardware drops.  Needs N % 8 == 0 and 2 M N < 2^31.

template <int ODT, int TM, int TN, int SHIFT, int FM0, int FM1, class V = i32x4>
__device__ __forceinline__ void epilogue_pass(const V (&acc)[TN / 16][TM / 16], uint8_t* region, int lane,
                                              int mw, int nw, int M, int N, const float* xs_lds,
                                              const float* ws_lds, const float* bias_lds,
                                              __amdgpu_buffer_rsrc_t orsrc, int m0, int n0) {
  static_assert(ODT == kBF16 || ODT == kF16, "16-bit outputs");
  constexpr int FN = TN / 16, RS = TN * 2 + 16, CPR = TN / 8, ROWS = (FM1 - FM0) * 16;
  constexpr int NIT = ROWS * CPR / 64;
  static_assert(ROWS * CPR % 64 == 0, "whole store instructions per pass");
  float xs[FM1 - FM0];
#pragma unroll
  for (int fm = FM0; fm < FM1; ++fm) xs[fm - FM0] = xs_lds[mw + fm * 16 + (lane & 15) - m0];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int nl = fn * 16 + 4 * (lane >> 4);
    const float4 w4 = *(const float4*)(ws_lds + (nw + nl - n0));
    const float4 b4 = *(const float4*)(bias_lds + (nw + nl - n0));
    const float wsv[4] = {w4.x, w4.y, w4.z, w4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
    for (int fm = FM0; fm < FM1; ++fm) {
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = ((acc_value<SHIFT>(acc[fn][fm][r]) * xs[fm - FM0]) * wsv[r]) + bv[r];
      const uint2 w = ODT == kBF16 ? make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]))
                                   : make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
      *(uint2*)(region + ((fm - FM0) * 16 + (lane & 15)) * RS + nl * 2) = w;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = it * 64 + lane, row = c / CPR, cc = c % CPR;
    const int m = mw + FM0 * 16 + row, n = nw + cc * 8;
    const uint4 v = *(const uint4*)(region + row * RS + cc * 16);
    const uint32_t off = (m < M && n < N) ? (uint32_t)((m * N + n) * 2) : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b128((u32x4){v.x, v.y, v.z, v.w}, orsrc, (int)off, 0, 0);
  }
  // the region's next writes (the next pass) come after these reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// The 16-bit epilogue of a wave's TM x TN corner held as 32 x 32 blocks
// (mfma_agpr32's layout): ((float(acc) * xs) * ws) + bias as in `epilogue`,
// staged through the wave's LDS region (TM rows of TN * 2 + 16 bytes) and
// written as range-checked 16-byte buffer stores.  Needs N % 8 == 0 and
// 2 M N < 2^31.
template <int ODT, int TM, int TN, int SHIFT>
__device__ __forceinline__ void epilogue32(const i32x16 (&acc)[TN / 32][TM / 32], uint8_t* region, int lane, int mw,
                                           int nw, int M, int N, const float* xs_lds, const float* ws_lds,
                                           const float* bias_lds, __amdgpu_buffer_rsrc_t orsrc, int m0, int n0) {
  static_assert(ODT == kBF16 || ODT == kF16, "16-bit outputs");
  constexpr int FN = TN / 32, FM = TM / 32, RS = TN * 2 + 16, CPR = TN / 8;
  constexpr int NIT = TM * CPR / 64;
  static_assert(TM * CPR % 64 == 0, "whole store instructions");
  float xs[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) xs[fm] = xs_lds[mw + fm * 32 + (lane & 31) - m0];
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = fn * 32 + 8 * q + 4 * (lane >> 5);
      const float4 w4 = *(const float4*)(ws_lds + (nw + nl - n0));
      const float4 b4 = *(const float4*)(bias_lds + (nw + nl - n0));
      const float wsv[4] = {w4.x, w4.y, w4.z, w4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (((float)(acc[fn][fm][4 * q + r] >> SHIFT) * xs[fm]) * wsv[r]) + bv[r];
        const uint2 w = ODT == kBF16 ? make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]))
                                     : make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
        *(uint2*)(region + (fm * 32 + (lane & 31)) * RS + nl * 2) = w;
      }
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int c = it * 64 + lane, row = c / CPR, cc = c % CPR;
    const int m = mw + row, n = nw + cc * 8;
    const uint4 v = *(const uint4*)(region + row * RS + cc * 16);
    const uint32_t off = (m < M && n < N) ? (uint32_t)((m * N + n) * 2) : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b128((u32x4){v.x, v.y, v.z, v.w}, orsrc, (int)off, 0, 0);
  }
}

// The 4-wave 256x256 kAgpr tile on v_mfma_i32_32x32x32_i8, one tile per
// workgroup, plain 16-bit epilogue (N % 8 == 0, 2 M N < 2^31).
template <int STAGES, int ODT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void w4a4_gemm_agpr32_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n) {
  using E = DmaEngine<256, 256, 2, 2, kAgpr, STAGES>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  E e(smem);

  const int tiles = tiles_m * tiles_n;
  int logical = blockIdx.x;
  const int per_xcd = tiles / kXcds;
  if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
  int m0, n0;
  tile_origin(logical, tiles_m, tiles_n, 256, 256, m0, n0);

  e.set_tile(act, wq, M, K, nblocks, kblocks, m0, n0);
  e.issue_epi(xscales, wscales, bias, M, N, m0, n0);
  i32x16 acc[E::FN32][E::FM32];
#pragma unroll
  for (int a = 0; a < E::FN32; ++a)
#pragma unroll
    for (int b = 0; b < E::FM32; ++b) acc[a][b] = (i32x16){};
  e.prologue(0, kblocks);
  e.body_agpr32(0, kblocks, acc);
  __syncthreads();  // all waves done with the LDS ring before it is reused for output staging
  const __amdgpu_buffer_rsrc_t orsrc =
      __builtin_amdgcn_make_buffer_rsrc(out, (short)0, (int)((int64_t)M * N * 2), 0x00020000);
  epilogue32<ODT, E::TM, E::TN, E::SHIFT>(acc, e.staging(), e.lane, m0 + e.wm * E::TM, n0 + e.wn * E::TN, M, N,
                                          e.epi_xs(), e.epi_ws(), e.epi_bias(), orsrc, m0, n0);
}

// Persistent form of the kAgpr data-parallel kernel for multi-round grids with
// the plain 16-bit epilogue: workgroup g runs tiles g, g + G, g + 2G, ... (G =
// gridDim.x, a multiple of the XCD count, so each tile keeps the XCD the
// one-tile-per-workgroup kernel gives it).  At a tile boundary the workgroup
// fetches the next tile's epilogue operands (into the other operand buffer)
// and first k-block (ring stage 0) before the current tile's epilogue, which
// stages its output through ring stages 1 and 2 in two passes; the next
// tile's k-blocks 1 and 2 follow once every wave is done with the staging.  So
// the first DMA's latency and the workgroup relaunch overlap the epilogue.
// The next tile's first wait (at most 2 x LPW DMAs in flight) retires block 0
// and everything issued before blocks 1 and 2, the output stores included.
// Arguments of the persistent kernel.  The kernel parks them in LDS and reads
// them back at each tile boundary, so they do not occupy scalar registers
// across the k-loop (kept live there, they spilled).
struct PersistArgs {
  const int8_t* act;
  const uint8_t* wq;
  const float* xscales;
  const float* wscales;
  const float* bias;
  void* out;
  int M, N, K, nblocks, kblocks, tiles_m, tiles_n;
};

// A wave-uniform value read back from LDS into scalar registers.
template <class T>
__device__ __forceinline__ T lds_uniform(const T& v) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "dword or qword");
  if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
  } else {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint64_t r = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)u) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(u >> 32)) << 32);
    return __builtin_bit_cast(T, r);
  }
}

template <int BM, int BN, int STAGES, int ODT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void w4a4_gemm_agpr_persist_kernel(
    PersistArgs args) {
  using E = DmaEngine<BM, BN, 2, 2, kAgpr, STAGES>;
  constexpr int FM = E::FM, P1 = (FM + 1) / 2;  // fragment rows of the first pass
  constexpr int RS = E::TN * 2 + 16;
  static_assert(E::NW * P1 * 16 * RS <= 2 * E::STAGE_BYTES, "two-pass staging fits ring stages 1 and 2");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES_2EPI];
  __shared__ PersistArgs la;
  E e(smem);

  const int tiles = args.tiles_m * args.tiles_n;
  int t = blockIdx.x, m0, n0;
  if (t >= tiles) return;  // the grid is rounded up to a multiple of the XCD count
  auto origin = [](int t, int tiles_m, int tiles_n, int& m0, int& n0) {
    const int tiles = tiles_m * tiles_n, per_xcd = tiles / kXcds;
    int logical = t;
    if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
    tile_origin(logical, tiles_m, tiles_n, BM, BN, m0, n0);
  };
  if (threadIdx.x == 0) la = args;  // published by the first k-block's barrier
  origin(t, args.tiles_m, args.tiles_n, m0, n0);
  e.set_tile(args.act, args.wq, args.M, args.K, args.nblocks, args.kblocks, m0, n0);
  e.issue_epi(args.xscales, args.wscales, args.bias, args.M, args.N, m0, n0);
  e.prologue(0, args.kblocks);
  int kblocks = args.kblocks;
  i32x4 acc[E::FN][FM];
  while (true) {
    // Opaque per tile: keeps the compiler from hoisting lane-derived addresses
    // out of the tile loop, where they would stay live across the k-loop.
    asm volatile("" : "+v"(e.lane), "+s"(kblocks));
#pragma unroll
    for (int a = 0; a < E::FN; ++a)
#pragma unroll
      for (int b = 0; b < FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};
    e.body_agpr(0, kblocks, acc, nullptr, 0);
    // every wave is done with the ring and the DMAs of this tile have landed
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int M = lds_uniform(la.M), N = lds_uniform(la.N);
    const int tiles_m = lds_uniform(la.tiles_m), tiles_n = lds_uniform(la.tiles_n);
    const int nt = t + (int)gridDim.x;
    const bool more = nt < tiles_m * tiles_n;
    const int cur = e.epi_buf;
    int nm0 = 0, nn0 = 0;
    if (more) {
      origin(nt, tiles_m, tiles_n, nm0, nn0);
      e.set_tile(lds_uniform(la.act), lds_uniform(la.wq), M, lds_uniform(la.K), lds_uniform(la.nblocks), kblocks,
                 nm0, nn0);
      e.epi_buf = cur ^ 1;
      e.issue_epi(lds_uniform(la.xscales), lds_uniform(la.wscales), lds_uniform(la.bias), M, N, nm0, nn0);
      e.issue(0, 0);
    }
    const __amdgpu_buffer_rsrc_t orsrc =
        __builtin_amdgcn_make_buffer_rsrc(lds_uniform(la.out), (short)0, (int)((int64_t)M * N * 2), 0x00020000);
    const int mw = m0 + e.wm * E::TM, nw = n0 + e.wn * E::TN;
    uint8_t* staging = smem + E::STAGE_BYTES + e.wave * (P1 * 16 * RS);
    const uint8_t* epi = smem + E::EPI_OFF + cur * E::EPI_BYTES;
    const float* xs_lds = (const float*)epi;
    const float* ws_lds = (const float*)(epi + (E::WS_OFF - E::EPI_OFF));
    const float* b_lds = (const float*)(epi + (E::BIAS_OFF - E::EPI_OFF));
    epilogue_pass<ODT, E::TM, E::TN, E::SHIFT, 0, P1>(acc, staging, e.lane, mw, nw, M, N, xs_lds, ws_lds, b_lds,
                                                      orsrc, m0, n0);
    epilogue_pass<ODT, E::TM, E::TN, E::SHIFT, P1, FM>(acc, staging, e.lane, mw, nw, M, N, xs_lds, ws_lds, b_lds,
                                                       orsrc, m0, n0);
    if (!more) break;
    // every wave is done with the staging area (ring stages 1 and 2)
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    e.issue(min(1, kblocks - 1), 1);
    e.issue(min(2, kblocks - 1), 2);
    t = nt;
    m0 = nm0;
    n0 = nn0;
  }
}

// ---- FP6 operands
//
// A code v in [-8, 7] is stored as the FP6 (e2m3) encoding of v/8: the
// subnormal with mantissa |v| for |v| <= 7 (a sign-magnitude field), -1.0 for
// -8.  The FP6 form of v_mfma_scale_f32_16x16x128_f8f6f4 with both operand
// scales 2^3 multiplies (v/8 * 8) (w/8 * 8) = v w exactly and accumulates in
// float32, exact while |sum| < 2^24 (K * 64 < 2^24 for every K below
// 262,144): the sums equal the int32 dots, and the epilogue sees the same
// values.  The instruction runs at twice the INT8 MFMA rate per cycle.
//
// Operand layout, the same for activations (rows) and weights (columns), K a
// multiple of 128: a k-block is 128 features in four 32-feature groups; a
// group's 32 six-bit codes (feature i at bits 6i..6i+5) form a 24-byte stream
// split into a 16-byte head and an 8-byte tail.  [K/128][ceil(R/16)][1536]:
// the 16 rows (columns) of a block, layout lane L = 16 g + r (row r, group g)
// holding its head at 16 L and its tail at 1024 + 8 L, i.e. the 6 dwords lane
// L of the MFMA operand takes.  A tile's k-block is one contiguous run of
// blocks, moved by whole 1 KB DMAs.
typedef int i32x6 __attribute__((ext_vector_type(6)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void mfma_fp6(f32x4& c, const i32x6& b, const i32x6& a, int scale) {
  asm volatile("v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0] cbsz:2 blgp:2"
               : "+a"(c)
               : "v"(b), "v"(a), "v"(scale)
               : "memory");
}

template <int FN, int FM>
__device__ __forceinline__ void mfma_drain_f(f32x4 (&acc)[FN][FM]) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) asm volatile("" : "+a"(acc[fn][fm]));
}

__device__ __forceinline__ i32x6 fp6_operand(const uint8_t* head, const uint8_t* tail) {
  const i32x4 h = *(const i32x4*)head;
  const i32x2 t = *(const i32x2*)tail;
  return (i32x6){h[0], h[1], h[2], h[3], t[0], t[1]};
}

// Compact FP6 weights: a weight whose codes lie in [-7, 7] has FP6 fields with
// both exponent bits zero, 4 bits of information each.  A lane's 32 fields
// are stored as four dwords i0..i3 of the 6-dword operand d0..d5:
//   i0 = (d0 & ~Z0) | (d2 & Z0), i1 = (d1 & ~Z1) | (d2 & Z1)  (i2, i3 from d3 .. d5)
// where Z0 and Z1 are the exponent bits of d0 and d1; d2's exponent bits are
// the positions in neither mask.  The expansion back is four bit operations
// per 16 fields, in inline asm so that the scheduler keeps it where the
// k-loop places it (between MFMAs) and the masks stay in SGPRs.
constexpr uint32_t kFp6cZ0 = 0x18618618u, kFp6cZ1 = 0x86186186u;

template <bool PAD = false>
__device__ __forceinline__ i32x6 fp6c_expand(const i32x4& i, uint32_t z0, uint32_t z1) {
  i32x6 d;
  asm volatile(
      "v_bfi_b32 %0, %8, 0, %6\n\t"      // d0 = i0 & ~Z0
      "v_bfi_b32 %1, %9, 0, %7\n\t"      // d1 = i1 & ~Z1
      "v_and_b32 %2, %9, %7\n\t"         // i1 & Z1
      "v_and_or_b32 %2, %6, %8, %2\n\t"  // d2 = (i0 & Z0) | (i1 & Z1)
      "v_bfi_b32 %3, %8, 0, %10\n\t"     // d3 = i2 & ~Z0
      "v_bfi_b32 %4, %9, 0, %11\n\t"     // d4 = i3 & ~Z1
      "v_and_b32 %5, %9, %11\n\t"        // i3 & Z1
      "v_and_or_b32 %5, %10, %8, %5"       // d5 = (i2 & Z0) | (i3 & Z1)
      : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3]), "=&v"(d[4]), "=&v"(d[5])
      : "v"(i[0]), "v"(i[1]), "s"(z0), "s"(z1), "v"(i[2]), "v"(i[3]));
  // wait states between these VALU writes and an MFMA that reads them one
  // instruction later (callers whose next reader is further away skip it)
  if constexpr (PAD) asm volatile("s_nop 2" ::: "memory");
  return d;
}

// The FP6 tile: BM x BN, waves 2 x WN, FN x FM 16 x 16 accumulator blocks per
// wave in the AGPRs; a 3-stage LDS ring of k-blocks (the tile's
// activation blocks, then its weight blocks).  Per k-block, one k-step of FN x
// FM MFMAs in two halves: half 0 (fragment rows 0 .. FM/2-1) reads the
// block's other activation fragments; a barrier publishes block i+1 and frees
// the block's stage; half 1 reads block i+1's weights (into the spare set) and
// first activation fragments, and issues the DMAs of block i+3.
//
// CW (compact weights): the weight blocks are 1024 bytes (the compact layout
// above).  Half 1 reads block i+1's weight fragments raw (16 bytes a lane);
// fragment 0 is expanded at the end of half 1, after its last use, and
// fragment fn >= 1 during half 0 of block i+1, which runs its MFMAs fragment
// by fragment (fn-major), so each expansion overlaps the MFMAs of fragment
// fn - 1.
//
// WN = 2: four waves, one a SIMD (up to 128 x 112 wave tiles).  WN = 4 (the
// 256 x 256, 128 x 256 and 128 x 192 tiles): eight waves, two a SIMD, with
// 128 x 64, 64 x 64 and 64 x 48 wave tiles (at most 128 AGPRs and 128 VGPRs);
// while one wave of a SIMD waits at the block barrier or on its fragment
// reads, the other's MFMAs run, and the activation blocks in LDS serve four
// wave columns instead of two.
template <int BM, int BN, bool CW = false, int WN = 2>
struct Fp6Engine {
  // A fourth ring stage on the 128-row compact tiles that run one workgroup per
  // CU: their block i+1 is published at block i's start, half a block earlier.
  static constexpr int NW = 2 * WN, STAGES = (CW && BM == 128 && BN > 128) ? 4 : 3;
  static constexpr int TM = BM / 2, TN = BN / WN, FM = TM / 16, FN = TN / 16, HM = FM / 2;
  static constexpr int WBLK = CW ? 1024 : 1536;  // bytes of one 16 x 128 weight block
  static constexpr int A_BYTES = (BM / 16) * 1536, B_BYTES = (BN / 16) * WBLK, STAGE_BYTES = A_BYTES + B_BYTES;
  // 1 KB DMA pieces per k-block; a wave issues APW + BPW of them (a count that
  // does not divide by the waves is padded with repeats of the last piece,
  // which rewrite the same bytes)
  static constexpr int A_DMAS = A_BYTES / 1024, B_DMAS = B_BYTES / 1024;
  static constexpr int APW = (A_DMAS + NW - 1) / NW, BPW = (B_DMAS + NW - 1) / NW, LPW = APW + BPW;
  static constexpr int XS_DMAS = (BM * 4 + 255) / 256, WS_DMAS = (BN * 4 + 255) / 256;
  static constexpr int EPI_DMAS = XS_DMAS + 2 * WS_DMAS;
  static constexpr int RS = TN * 2 + 16, STAGING = TM * RS;
  // the epilogue operands sit past both the ring and the output staging (which
  // outgrows the ring of compact-weight tiles)
  static constexpr int EPI_OFF = STAGES * STAGE_BYTES > NW * STAGING ? STAGES * STAGE_BYTES : NW * STAGING;
  static constexpr int WS_OFF = EPI_OFF + XS_DMAS * 256, BIAS_OFF = WS_OFF + WS_DMAS * 256;
  static constexpr int SMEM_BYTES = EPI_OFF + EPI_DMAS * 256;
  static_assert(A_BYTES % 1024 == 0 && B_BYTES % 1024 == 0, "whole DMA pieces (BM and BN multiples of 32)");
  static_assert(FM % 2 == 0 && NW * STAGING <= EPI_OFF && SMEM_BYTES <= 160 * 1024, "LDS of one CU");
  static_assert((STAGES - 1) * LPW <= 63, "vmcnt counts at most 63 DMAs");

  uint8_t* smem;
  uint32_t smem_addr;
  int lane, wave, wm, wn;
  i32x4_sgpr ra, rw;
  uint32_t vl, a_kstride, w_kstride;

  __device__ __forceinline__ explicit Fp6Engine(uint8_t* s) : smem(s) {
    smem_addr = (uint32_t)(uintptr_t)s;
    lane = threadIdx.x & 63;
    wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    wm = wave / WN;
    wn = wave % WN;
  }

  __device__ __forceinline__ void issue_epi(const float* xscales, const float* wscales, const float* bias, int M,
                                            int N, int m0, int n0) {
    for (int d = wave; d < EPI_DMAS; d += NW) {
      const int arr = d < XS_DMAS ? 0 : d < XS_DMAS + WS_DMAS ? 1 : 2;
      const int q = d - (arr == 0 ? 0 : arr == 1 ? XS_DMAS : XS_DMAS + WS_DMAS);
      const int off = arr == 0 ? EPI_OFF : arr == 1 ? WS_OFF : BIAS_OFF;
      const float* base = arr == 0 ? xscales + m0 : arr == 1 ? wscales + n0 : (bias ? bias + n0 : wscales);
      const int count = arr == 0 ? M - m0 : (arr == 1 || bias) ? N - n0 : 0;
      const i32x4_sgpr r = buffer_rsrc(base, (uint32_t)count * 4u);
      dma4(r, (uint32_t)(q * 256 + lane * 4), smem_addr + (uint32_t)(off + q * 256));
    }
  }

  // Piece j of a k-block: bytes 1024 j .. of the tile's activation blocks
  // (pieces 0 .. A_DMAS-1) or weight blocks.  Blocks past the last row
  // (column) block of the last k-block read as zero; other blocks past the
  // tile's edge read the next k-block's first blocks, which only reach
  // accumulators of rows (columns) that are never stored.
  __device__ __forceinline__ void set_tile(const uint8_t* act, const uint8_t* wq, int M, int K, int nblocks,
                                           int m0, int n0) {
    const int kblocks = K / 128, mblocks = (M + 15) / 16;
    ra = buffer_rsrc(act + (int64_t)(m0 / 16) * 1536, (uint32_t)(((int64_t)kblocks * mblocks - m0 / 16) * 1536));
    rw = buffer_rsrc(wq + (int64_t)(n0 / 16) * WBLK, (uint32_t)(((int64_t)kblocks * nblocks - n0 / 16) * WBLK));
    vl = (uint32_t)lane * 16u;
    a_kstride = (uint32_t)mblocks * 1536u;
    w_kstride = (uint32_t)nblocks * (uint32_t)WBLK;
  }

  __device__ __forceinline__ void issue_piece(int kb, int stage, int idx) {
    const uint32_t base = smem_addr + (uint32_t)(stage * STAGE_BYTES);
    if (idx < APW) {
      const uint32_t j = (uint32_t)min(wave * APW + idx, A_DMAS - 1);
      uint32_t so = j * 1024u + (uint32_t)kb * a_kstride;
      asm volatile("" : "+s"(so));
      dma16(ra, vl + so, base + j * 1024u);
    } else {
      const uint32_t j = (uint32_t)min(wave * BPW + idx - APW, B_DMAS - 1);
      uint32_t so = j * 1024u + (uint32_t)kb * w_kstride;
      asm volatile("" : "+s"(so));
      dma16(rw, vl + so, base + (uint32_t)A_BYTES + j * 1024u);
    }
  }

  __device__ __forceinline__ void prologue(int n) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s)
#pragma unroll
      for (int p = 0; p < LPW; ++p) issue_piece(min(s, n - 1), s, p);
  }

  __device__ __forceinline__ i32x6 read_a(int stage, int fm) const {
    const uint8_t* blk = smem + stage * STAGE_BYTES + (wm * FM + fm) * 1536;
    return fp6_operand(blk + 16 * lane, blk + 1024 + 8 * lane);
  }
  __device__ __forceinline__ i32x6 read_b(int stage, int fn) const {
    const uint8_t* blk = smem + stage * STAGE_BYTES + A_BYTES + (wn * FN + fn) * 1536;
    return fp6_operand(blk + 16 * lane, blk + 1024 + 8 * lane);
  }
  __device__ __forceinline__ i32x4 read_b_raw(int stage, int fn) const {
    return *(const i32x4*)(smem + stage * STAGE_BYTES + A_BYTES + (wn * FN + fn) * 1024 + 16 * lane);
  }

  // One quarter of a compact fragment's expansion (two instructions) into d.
  template <int PART>
  __device__ __forceinline__ static void expand_part(const i32x4& r, i32x6& d, uint32_t z0, uint32_t z1) {
    int x, y;
    if constexpr (PART == 0) {
      asm volatile("v_bfi_b32 %0, %2, 0, %4\n\tv_bfi_b32 %1, %3, 0, %5"
                   : "=&v"(x), "=&v"(y) : "s"(z0), "s"(z1), "v"(r[0]), "v"(r[1]));
      d[0] = x, d[1] = y;
    } else if constexpr (PART == 1) {
      asm volatile("v_and_b32 %0, %2, %4\n\tv_and_or_b32 %0, %3, %1, %0"
                   : "=&v"(x) : "s"(z0), "s"(z1), "v"(r[0]), "v"(r[1]));
      d[2] = x;
    } else if constexpr (PART == 2) {
      asm volatile("v_bfi_b32 %0, %2, 0, %4\n\tv_bfi_b32 %1, %3, 0, %5"
                   : "=&v"(x), "=&v"(y) : "s"(z0), "s"(z1), "v"(r[2]), "v"(r[3]));
      d[3] = x, d[4] = y;
    } else {
      asm volatile("v_and_b32 %0, %2, %4\n\tv_and_or_b32 %0, %3, %1, %0"
                   : "=&v"(x) : "s"(z0), "s"(z1), "v"(r[2]), "v"(r[3]));
      d[5] = x;
    }
  }

  // Compact weights: k-block i (ring stage st) with expanded fragments b; block
  // i+1's raw fragments are read and expanded into bn a quarter fragment (two
  // instructions) at a time between later MFMAs, so the MFMA pipe never waits
  // on a burst of expansions.  On the 256-row tiles (FM = 8) half 1 has room
  // for them all: it reads block i+1's raw fragments first (its stage is
  // published by the barrier between the halves) and expands them after MFMA
  // kT0 on.  The 128-row tiles (FM = 4) need both halves (EARLY): a second
  // barrier at the block's start publishes block i+1's stage, half 0 reads the
  // raw fragments, and the expansions run from half 0's MFMA kT0 to the end.
  static constexpr bool kEarly = HM == 2;
  static constexpr int kT0 = FN + 2;  // first MFMA gap of the expansions (the raw reads landed)
  static constexpr int kGaps = (kEarly ? 2 : 1) * HM * FN - kT0;
  // part k of the 4 FN goes after MFMA kT0 + floor(k kGaps / (4 FN)) (counting half 0's
  // MFMAs first when early); part_lo(t) is the first part at or after gap t
  static constexpr int part_lo(int t) {
    const int d = t - kT0;
    return d <= 0 ? 0 : (d * 4 * FN + kGaps - 1) / kGaps;
  }
  static_assert(kGaps > 0 && (4 * FN + kGaps - 1) / kGaps <= 3, "at most three parts a gap");

  // the expansion parts after MFMA g (0 .. 2 HM FN - 1 across the two halves)
  __device__ __forceinline__ void expand_parts(int g, i32x4 (&raw)[FN], i32x6 (&bn)[FN], uint32_t z0,
                                               uint32_t z1) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int k = part_lo(g) + j;
      if (g >= kT0 && k < part_lo(g + 1) && k < 4 * FN) {
        if (k % 4 == 0) expand_part<0>(raw[k / 4], bn[k / 4], z0, z1);
        if (k % 4 == 1) expand_part<1>(raw[k / 4], bn[k / 4], z0, z1);
        if (k % 4 == 2) expand_part<2>(raw[k / 4], bn[k / 4], z0, z1);
        if (k % 4 == 3) expand_part<3>(raw[k / 4], bn[k / 4], z0, z1);
      }
    }
  }

  __device__ __forceinline__ void block_c2(int st, int nst, int dma_kb, const i32x6 (&b)[FN], i32x6 (&bn)[FN],
                                           i32x4 (&raw)[FN], i32x6 (&a)[FM], f32x4 (&acc)[FN][FM], int scale,
                                           uint32_t z0, uint32_t z1) {
    constexpr int NS = HM * FN;
    if constexpr (kEarly) {
      wait_vmcnt<(STAGES - 2) * LPW>();  // block i+1 landed (later blocks' DMAs may be in flight)
      __builtin_amdgcn_s_barrier();
    }
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int fm = t / FN, fn = t % FN;
      mfma_fp6(acc[fn][fm], b[fn], a[fm], scale);
      if (t % 2 == 1 && t / 2 < HM) a[HM + t / 2] = read_a(st, HM + t / 2);
      if constexpr (kEarly) {
        if (t < FN) raw[t] = read_b_raw(nst, t);
        expand_parts(t, raw, bn, z0, z1);
      }
    }
#pragma unroll
    for (int i = 0; i < HM; ++i) asm volatile("" ::"v"(a[i]));
    wait_vmcnt<(STAGES - 2) * LPW>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int fm = HM + t / FN, fn = t % FN;
      mfma_fp6(acc[fn][fm], b[fn], a[fm], scale);
      if (!kEarly && t < FN) raw[t] = read_b_raw(nst, t);
      if (t >= FN && t < FN + HM) a[t - FN] = read_a(nst, t - FN);
#pragma unroll
      for (int p = 0; p < LPW; ++p)
        if (t == (p * NS) / LPW) issue_piece(dma_kb, st, p);
      expand_parts(kEarly ? NS + t : t, raw, bn, z0, z1);
    }
    // The MFMA reads its operand registers over its passes: the half's
    // fragments (b included) stay live to its end, so no temporary of the
    // expansions lands in the registers of an MFMA issued just before it.
#pragma unroll
    for (int i = HM; i < FM; ++i) asm volatile("" ::"v"(a[i]));
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) asm volatile("" ::"v"(b[fn]));
  }

  // k-block i (ring stage st) with weight fragments b; bn receives block i+1's.
  __device__ __forceinline__ void block(int st, int nst, int dma_kb, const i32x6 (&b)[FN], i32x6 (&bn)[FN],
                                        i32x6 (&a)[FM], f32x4 (&acc)[FN][FM], int scale) {
    constexpr int NS = HM * FN;  // MFMAs per half
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int fm = t / FN, fn = t % FN;
      mfma_fp6(acc[fn][fm], b[fn], a[fm], scale);
      if (t % 2 == 1 && t / 2 < HM) a[HM + t / 2] = read_a(st, HM + t / 2);
    }
    // the half's fragments stay live to its end, so no read of this half lands
    // in the registers of an MFMA issued just before it
#pragma unroll
    for (int i = 0; i < HM; ++i) asm volatile("" ::"v"(a[i]));
    wait_vmcnt<(STAGES - 2) * LPW>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int t = 0; t < NS; ++t) {
      const int fm = HM + t / FN, fn = t % FN;
      mfma_fp6(acc[fn][fm], b[fn], a[fm], scale);
      if (t < FN) bn[t] = read_b(nst, t);
      if (t >= FN && t < FN + HM) a[t - FN] = read_a(nst, t - FN);
#pragma unroll
      for (int p = 0; p < LPW; ++p)
        if (t == (p * NS) / LPW) issue_piece(dma_kb, st, p);
    }
#pragma unroll
    for (int i = HM; i < FM; ++i) asm volatile("" ::"v"(a[i]));
  }

  __device__ __forceinline__ void run(int n, f32x4 (&acc)[FN][FM]) {
    static_assert(LPW <= 2 * FN * HM, "DMA pieces fit the half");
    const int scale = (int)0x82828282u;  // E8M0 scales of 2^3 (one byte per 32-feature group)
    if constexpr (CW) {
      const uint32_t z0 = __builtin_amdgcn_readfirstlane(kFp6cZ0), z1 = __builtin_amdgcn_readfirstlane(kFp6cZ1);
      i32x6 a[FM], b[FN];
      i32x4 raw[FN];
      wait_vmcnt<(STAGES - 1) * LPW>();  // block 0 (and the epilogue operands) landed
      __builtin_amdgcn_s_barrier();
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) raw[fn] = read_b_raw(0, fn);
#pragma unroll
      for (int fm = 0; fm < HM; ++fm) a[fm] = read_a(0, fm);
      const int last = n - 1;
      int st = 0;
      auto nxt = [](int s) { return s + 1 == STAGES ? 0 : s + 1; };
      {
        i32x6 b1[FN];
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) b[fn] = fp6c_expand(raw[fn], z0, z1);
        asm volatile("s_nop 4" ::: "memory");
        int i = 0;
        for (; i + 1 < n; i += 2) {
          block_c2(st, nxt(st), min(i + STAGES, last), b, b1, raw, a, acc, scale, z0, z1);
          st = nxt(st);
          block_c2(st, nxt(st), min(i + 1 + STAGES, last), b1, b, raw, a, acc, scale, z0, z1);
          st = nxt(st);
        }
        if (i < n) block_c2(st, nxt(st), min(i + STAGES, last), b, b1, raw, a, acc, scale, z0, z1);
      }
      mfma_drain_f(acc);
      wait_vmcnt<0>();
      return;
    }
    i32x6 a[FM], b0[FN], b1[FN];
    wait_vmcnt<(STAGES - 1) * LPW>();  // block 0 (and the epilogue operands) landed
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) b0[fn] = read_b(0, fn);
#pragma unroll
    for (int fm = 0; fm < HM; ++fm) a[fm] = read_a(0, fm);
    const int last = n - 1;
    int st = 0, i = 0;
    auto nxt = [](int s) { return s + 1 == STAGES ? 0 : s + 1; };
    for (; i + 1 < n; i += 2) {
      block(st, nxt(st), min(i + STAGES, last), b0, b1, a, acc, scale);
      st = nxt(st);
      block(st, nxt(st), min(i + 1 + STAGES, last), b1, b0, a, acc, scale);
      st = nxt(st);
    }
    if (i < n) block(st, nxt(st), min(i + STAGES, last), b0, b1, a, acc, scale);
    mfma_drain_f(acc);
    wait_vmcnt<0>();
  }
};

// The FP6 GEMM, one BM x BN tile per workgroup of 2 WN waves, with the
// epilogue of every W4A4 kernel (16-bit or float32 outputs, optional gated
// residual).  Two waves a SIMD for the 128 x 128 tile (two workgroups a CU)
// and the 8-wave tiles.
template <int BM, int BN, int ODT, bool CW, int WN>
__global__ __launch_bounds__(WN * 128) __attribute__((amdgpu_waves_per_eu(WN == 4 ? 2 : 1, BM * BN <= 128 * 128 || WN == 4 ? 2 : 1))) void w4a4_gemm_fp6_kernel(
    const uint8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int tiles_m, int tiles_n, GatedResidual gr) {
  using E = Fp6Engine<BM, BN, CW, WN>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  E e(smem);
  const int tiles = tiles_m * tiles_n;
  int logical = blockIdx.x;
  const int per_xcd = tiles / kXcds;
  if (logical < per_xcd * kXcds) logical = (logical % kXcds) * per_xcd + logical / kXcds;
  int m0, n0;
  tile_origin(logical, tiles_m, tiles_n, BM, BN, m0, n0);
  const int kblocks = K / 128;
  e.set_tile(act, wq, M, K, nblocks, m0, n0);
  e.issue_epi(xscales, wscales, bias, M, N, m0, n0);
  f32x4 acc[E::FN][E::FM];
#pragma unroll
  for (int a = 0; a < E::FN; ++a)
#pragma unroll
    for (int b = 0; b < E::FM; ++b) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};
  e.prologue(kblocks);
  e.run(kblocks, acc);
  __syncthreads();  // ring -> output staging
  epilogue<ODT, E::TM, E::TN, 0, true, f32x4, true>(acc, smem + e.wave * E::STAGING, e.lane, m0 + e.wm * E::TM,
                                       n0 + e.wn * E::TN, M, N, (const float*)(smem + E::EPI_OFF),
                                       (const float*)(smem + E::WS_OFF), (const float*)(smem + E::BIAS_OFF), out, gr,
                                       m0, n0);
}

// ---- stream-K
//
// Workspace (device memory, zero-filled once before its first launch; every
// launch leaves it ready for the next launch that uses it):
//   int32 word 32 g          ticket counter of workgroup group g (one group per XCD)
//   int32 word 256 + 32 g    finished-workgroup counter of group g
//   int32 word 512 + 32 g    generation of group g, advanced by the group's last workgroup
//   int32 word 768           error word: nonzero once an owner's bounded wait gave up
//   int32 words [1024, 1024+G*NW) partial-ready flag of each (workgroup slot, wave):
//                            the generation tag (generation + 1) of the launch that raised it
//   bytes [kSkPartialOffset, ...)  one int32 partial tile per workgroup slot
// Each counter has a 128-byte line to itself: every workgroup of the launch
// performs two device-scope atomics on its group's counters, and atomics on
// one line are serialized.  Flags are never cleared: a launch waits for its
// own generation's tag, so a flag left by an earlier launch never matches.
// Launches that use one workspace must not overlap in time (one stream).
constexpr int kSkLineWords = 32;
constexpr int kSkDoneWord = kXcds * kSkLineWords;
constexpr int kSkGenWord = 2 * kSkDoneWord;
constexpr int kSkErrorWord = 3 * kSkDoneWord;
constexpr int kSkCtlWords = 4 * kSkDoneWord;
constexpr int64_t kSkPartialOffset = 32768;
constexpr int kSkMaxGrid = 512;  // <= 64 workgroups per group: one lane per contributor when polling
constexpr int kSkMaxWaves = 8;
static_assert(kSkCtlWords + kSkMaxGrid * kSkMaxWaves <= kSkPartialOffset / 4, "flags overflow the control block");
constexpr int kSkGenMask = 0x3fffffff;
constexpr int kSkSpinLimit = 1 << 22;  // ~1 s of s_sleep 4 polls: a lost flag ends the wait instead of hanging

// Partials and flags are exchanged with device-scope (sc1) accesses only:
// each is coherent across CUs (and XCDs) by itself, and order is kept by
// waiting for the partial's stores to complete (vmcnt 0) before its flag is
// raised and by issuing the loads only after the flag was seen.  Acquire /
// release fences would also work but write back and invalidate the whole L2
// of the XCD, which evicts the operand tiles every other workgroup is using.
// The partial's loads are issued through asm: as C++ atomics the compiler
// waits for each load before issuing the next (one round trip per 8 bytes).
// Its stores stay C++ atomics (64-bit): the compiler must see every store to
// keep the wait state a VMEM store of more than 64 bits needs before its data
// registers are rewritten, which it cannot do for a store inside asm.
// (load_dev16 is in convrot_device.h.)
static_assert(kSkCtlWords + kSkMaxGrid * kSkMaxWaves <= (int)(kW4a16CounterOffset / 4),
              "the W4A16 split-K counters follow the stream-K flags in the control block");

// One wave's partial tile: fragment f = fn * FM + fm at byte 1024 f + 16 lane.
template <int FN, int FM>
__device__ __forceinline__ void sk_store_partial(uint8_t* dst, int lane, const i32x4 (&acc)[FN][FM]) {
  uint64_t* p = (uint64_t*)(dst + lane * 16);
#pragma unroll
  for (int fn = 0; fn < FN; ++fn)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const i32x4 a = acc[fn][fm];
      uint64_t* q = p + (fn * FM + fm) * 128;
      __hip_atomic_store(q, (uint64_t)(uint32_t)a[0] | ((uint64_t)(uint32_t)a[1] << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(q + 1, (uint64_t)(uint32_t)a[2] | ((uint64_t)(uint32_t)a[3] << 32), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
}

// acc += one wave's partial tile: loads in batches of up to 16 fragments
// (8 beside a 32- or 64-fragment accumulator), one wait per batch.
template <int FN, int FM>
__device__ __forceinline__ void sk_add_partial(const uint8_t* src, int lane, i32x4 (&acc)[FN][FM]) {
  constexpr int NF = FN * FM;
  constexpr int BATCH = NF >= 32 ? 8 : NF;
  static_assert(NF % 4 == 0 && NF % BATCH == 0, "fragment batches");
  const uint8_t* p = src + lane * 16;
#pragma unroll
  for (int b = 0; b < NF; b += BATCH) {
    i32x4 v[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; j += 4) {
      const uint8_t* q = p + (b + j) * 1024;
      v[j] = load_dev16<0>(q);
      v[j + 1] = load_dev16<1024>(q);
      v[j + 2] = load_dev16<2048>(q);
      v[j + 3] = load_dev16<3072>(q);
    }
    wait_vmcnt<0>();
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      asm volatile("" : "+v"(v[j]));  // the adds stay behind the wait
      acc[(b + j) / FM][(b + j) % FM] += v[j];
    }
  }
}

// Lane i < n polls flag first[i * stride] until it holds `tag` (all lanes in
// parallel), at most spin_limit times.  Returns false (wave-uniform) when some
// flag was not seen: the caller then reports the failure and poisons its
// output instead of proceeding with a partial missing.
__device__ __forceinline__ bool sk_wait_flags(const int* first, int stride, int n, int lane, int tag,
                                              int spin_limit) {
  const int* f = first + (int64_t)lane * stride;
  bool seen = lane >= n;
  for (int it = 0; it < spin_limit; ++it) {
    if (!seen) seen = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == tag;
    if (__ballot(!seen) == 0) break;
    __builtin_amdgcn_s_sleep(4);
  }
  return __ballot(!seen) == 0;
}

// Arguments of a stream-K launch beyond the GEMM's own.
struct SkArgs {
  uint8_t* work;   // workspace (layout above)
  int min_iters;   // shortest stream-K range, in k-blocks
  int spin_limit;  // polls of an owner's bounded wait
};

// The persistent stream-K GEMM (Osama et al., "Stream-K: Work-centric
// Parallel Decomposition for Dense Matrix-Matrix Multiplication on the GPU",
// 2023), in its data-parallel + stream-K hybrid form, run per XCD, for the
// engine E (the 8-wave tiles or the 4-wave AGPR tile).
//
// The grid is G = 8 P workgroups; workgroup b belongs to group b % 8 (the XCD
// it is dispatched to) and takes a ticket 0..P-1 inside its group at start,
// so ticket order is start order.  Group x owns a contiguous run of Tx tiles
// of the grouped tile order (the same tiles the data-parallel kernel gives
// XCD x).  When Tx is not a multiple of P, all but the last one-to-two rounds
// of tiles run whole (data-parallel) and the remaining tiles' k-blocks are
// split into psk contiguous ranges, one per ticket.  Each workgroup walks its
// range from the top down, so the piece holding a tile's last k-blocks --
// whose workgroup owns the tile -- is the last piece that workgroup runs,
// while every other piece of the tile is the first stream-K piece of its
// (lower-ticket) workgroup.  Non-owners store their int32 partial sums and
// raise one flag per wave; each wave of the owner waits for the matching
// waves of the lower tickets that share its tile, adds their partials
// (integer addition: the result is bit-identical to a single pass) and the
// workgroup runs the fused epilogue.  Waits only ever point at lower tickets,
// i.e. at workgroups that have already started and that wait only on lower
// tickets themselves, so the kernel finishes whatever the residency.  The
// waits are bounded all the same: an owner that gives up sets the error word
// and writes NaN over its tile.
template <class E, int ODT>
__device__ __forceinline__ void sk_items(uint8_t* smem, int* s_shared, const int8_t* __restrict__ act,
                                         const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
                                         const float* __restrict__ wscales, const float* __restrict__ bias,
                                         void* __restrict__ out, int M, int N, int K, int nblocks, int kblocks,
                                         int tiles_m, int tiles_n, const SkArgs& ska, const GatedResidual& gr) {
  constexpr int FN = E::FN, FM = E::FM, NW = E::NW, BM = E::kBM, BN = E::kBN;
  static_assert(NW <= kSkMaxWaves, "flag block sized for 8 waves");
  int* ctl = (int*)ska.work;
  int* flags = ctl + kSkCtlWords;
  uint8_t* partials = ska.work + kSkPartialOffset;
  const int group = blockIdx.x % kXcds;
  const int P = gridDim.x / kXcds;
  if (threadIdx.x == 0) {
    s_shared[0] = atomicAdd(&ctl[group * kSkLineWords], 1);
    s_shared[1] = (__hip_atomic_load(&ctl[kSkGenWord + group * kSkLineWords], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) &
                   kSkGenMask) + 1;
  }
  __syncthreads();
  const int p = __builtin_amdgcn_readfirstlane(s_shared[0]);
  const int tag = __builtin_amdgcn_readfirstlane(s_shared[1]);
  // (constructed after the ticket: built before the barrier above, this
  // compiler loses track of the engine's wave-uniform DMA operands)
  E e(smem);

  const int tiles = tiles_m * tiles_n;
  const int base = tiles / kXcds, extra = tiles % kXcds;
  const int tb = group * base + min(group, extra);
  const int tx = base + (group < extra ? 1 : 0);
  const int rounds = tx / P, rem = tx % P;
  const int dp = rem == 0 ? tx : (rounds > 0 ? (rounds - 1) * P : 0);

  // Work items of this workgroup, in order: whole tiles p, p+P, ... < dp,
  // then the pieces of its stream-K range [lo, hi) from the top down.
  // (Range arithmetic fits 32 bits: fewer than 2P tiles of <= 512 k-blocks.)
  const int sk_iters = (tx - dp) * kblocks;
  const int psk = min(P, max(1, sk_iters / max(1, ska.min_iters)));
  const bool in_sk = sk_iters > 0 && p < psk;
  const int lo = in_sk ? sk_iters * p / psk : 0;
  int hi = in_sk ? sk_iters * (p + 1) / psk : 0;
  int next_dp = p;
  auto next_item = [&](int& t, int& k0, int& k1) {
    if (next_dp < dp) {
      t = next_dp;
      k0 = 0;
      k1 = kblocks;
      next_dp += P;
      return true;
    }
    if (hi > lo) {
      const int ts = (hi - 1) / kblocks;
      const int seg = max(lo, ts * kblocks);
      t = dp + ts;
      k0 = seg - ts * kblocks;
      k1 = hi - ts * kblocks;
      hi = seg;
      return true;
    }
    return false;
  };

  i32x4 acc[FN][FM];
  int t = 0, k0 = 0, k1 = 0;
  bool have = next_item(t, k0, k1);
  bool prefetched = false;  // the item's tile is set and its prologue DMAs issued
  int* pending = nullptr;   // this wave's partial-ready flag, raised by the next body
  while (have) {
    // Opaque per item: keeps the compiler from hoisting lane-derived epilogue
    // and partial addresses out of the loop, where they would stay live
    // (and spill) across the MFMA pipeline.
    asm volatile("" : "+v"(e.lane));
    int m0, n0;
    tile_origin(tb + t, tiles_m, tiles_n, BM, BN, m0, n0);
    if (!prefetched) {
      e.set_tile(act, wq, M, K, nblocks, kblocks, m0, n0);
      e.issue_epi(xscales, wscales, bias, M, N, m0, n0);
      e.prologue(k0, k1 - k0);
    }
#pragma unroll
    for (int a = 0; a < FN; ++a)
#pragma unroll
      for (int b = 0; b < FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};
    e.body_any(k0, k1 - k0, acc, pending, tag);
    pending = nullptr;

    int nt = 0, nk0 = 0, nk1 = 0;
    const bool more = next_item(nt, nk0, nk1);
    prefetched = false;
    // Partial tile of slot s: BM * BN * 4 bytes at partials + s * BM * BN * 4.
    const int64_t wave_off = (int64_t)e.wave * (FN * FM * 1024);
    if (k1 < kblocks) {
      // Not the tile's last k-blocks: publish the partial sums for the owner.
      // The stores go out first, then the next item's first DMAs, and the
      // next body raises the flag once its first wait has retired both (so
      // the store round trip overlaps the DMA one and the MFMAs after it).
      sk_store_partial<FN, FM>(partials + (int64_t)(group * P + p) * (BM * BN * 4) + wave_off, e.lane, acc);
      int* flag = &flags[(group * P + p) * NW + e.wave];
      if (more) {
        __syncthreads();  // every wave done reading the ring
        int nm0, nn0;
        tile_origin(tb + nt, tiles_m, tiles_n, BM, BN, nm0, nn0);
        e.set_tile(act, wq, M, K, nblocks, kblocks, nm0, nn0);
        e.issue_epi(xscales, wscales, bias, M, N, nm0, nn0);
        e.prologue(nk0, nk1 - nk0);
        prefetched = true;
        pending = flag;
      } else {
        wait_vmcnt<0>();
        if (e.lane == 0) __hip_atomic_store(flag, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      bool ok = true;
      if (k0 > 0) {
        // Lower tickets qf .. p-1 hold the tile's earlier k-blocks; ticket q's
        // range starts at sk_iters * q / psk.
        const int tstart = (t - dp) * kblocks;
        int qf = p - 1;
        while (sk_iters * qf / psk > tstart) --qf;
        ok = sk_wait_flags(&flags[(group * P + qf) * NW + e.wave], NW, p - qf, e.lane, tag, ska.spin_limit);
        if (ok) {
          for (int q = qf; q < p; ++q)
            sk_add_partial<FN, FM>(partials + (int64_t)(group * P + q) * (BM * BN * 4) + wave_off, e.lane, acc);
        } else if (e.lane == 0) {
          __hip_atomic_store(&ctl[kSkErrorWord], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      __syncthreads();  // ring -> epilogue staging
      epilogue<ODT, E::TM, E::TN, E::SHIFT, true>(acc, e.staging(), e.lane, m0 + e.wm * E::TM, n0 + e.wn * E::TN,
                                                  M, N, e.epi_xs(), e.epi_ws(), e.epi_bias(), out, gr, m0, n0,
                                                  !ok);
      __syncthreads();  // staging -> next item's DMA
    }
    t = nt;
    k0 = nk0;
    k1 = nk1;
    have = more;
  }

  // The last workgroup of the group to finish rearms the ticket counters and
  // advances the generation.
  if (threadIdx.x == 0) {
    if (atomicAdd(&ctl[kSkDoneWord + group * kSkLineWords], 1) == P - 1) {
      __hip_atomic_store(&ctl[group * kSkLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl[kSkDoneWord + group * kSkLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl[kSkGenWord + group * kSkLineWords], tag & kSkGenMask, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <int BM, int BN, int WM, int WN, int PIPE, int STAGES, int ODT>
__global__ __launch_bounds__(WM* WN * 64) void w4a4_gemm_sk_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, SkArgs ska, GatedResidual gr) {
  using E = DmaEngine<BM, BN, WM, WN, PIPE, STAGES>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  __shared__ int s_shared[2];
  sk_items<E, ODT>(smem, s_shared, act, xscales, wq, wscales, bias, out, M, N, K, nblocks, kblocks, tiles_m, tiles_n,
                   ska, gr);
}

// The stream-K kernel of the 4-wave AGPR 256x256 tile (512 registers per wave).
template <int STAGES, int ODT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void w4a4_gemm_agpr_sk_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, SkArgs ska, GatedResidual gr) {
  using E = DmaEngine<256, 256, 2, 2, kAgpr, STAGES>;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  __shared__ int s_shared[2];
  sk_items<E, ODT>(smem, s_shared, act, xscales, wq, wscales, bias, out, M, N, K, nblocks, kblocks, tiles_m, tiles_n,
                   ska, gr);
}

// ---- host side: plan choice, stream-K workspace, launches

struct Tile {
  int bm, bn, wm, wn;
  int stages;  // LDS ring depth of the DMA kernels
};

struct Plan {
  Tile t;
  bool sk;        // stream-K kernel (else one workgroup per tile)
  int grid;       // stream-K grid size (multiple of 8)
  int min_iters;  // shortest stream-K range, in k-blocks
};

}  // namespace

int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

namespace {

// Candidate tiles with the relative MFMA efficiency each sustains in steady
// state on MI355X, in units of the 4-wave 256x256 tile (accumulator in the
// AGPRs, software-pipelined k-steps), which measured 2-13 % faster than the
// 8-wave 256x256 tile on every FLUX shape at M = 1536 and 4608.  The 8-wave
// tile moves half the L2 bytes per MFMA of 128x128 but runs one workgroup per
// CU; 128x128 fits two per CU.  `sk` marks the tiles the stream-K kernel runs
// well: the 8-wave 256x256 one spills registers inside its k-loop there,
// 128x128 pieces are too short, and the 4-wave 256x256 stream-K kernel ran
// 1.4-2.8x slower than the data-parallel one on every FLUX shape timed
// (M = 1024 .. 4608), and 2x slower than 128x256 stream-K at 1536x12288->3072.
//
// The 192x128 tile moves more L2 bytes per MFMA than the 256x256 ones and
// sustains 0.69 of the 4-wave tile's rate with every CU busy, but 0.77 when
// its grid is a single round that leaves CUs idle (1536 tokens: 192 tiles at
// N = 3072).
//
// The 4-wave 288x192 tile (6 x 9 fragments per wave, data-parallel only) moves
// the same 48 KB per k-block as 256x256 for 0.84 of its MFMAs; at 4608 tokens
// its grid is exactly one workgroup per CU for every N multiple of 3072/16,
// where 256x256 leaves 40 CUs idle (N = 3072) or a 3/8-full last round.
struct Cand {
  Tile t;
  int per_cu;
  double eff;
  double eff_partial;  // eff when the grid is one round of fewer tiles than CUs
  bool sk;
  bool dma_only;   // no register-staged (packed-activation) variant
  bool no_sk = false;  // no stream-K kernel
};
constexpr Cand kCands[7] = {{{256, 256, 2, 2, 3}, 1, 1.0, 1.0, false, true},
                            {{256, 256, 2, 4, 3}, 1, 0.92, 0.92, false, false},
                            {{128, 256, 2, 4, 4}, 1, 0.79, 0.79, true, false},
                            {{256, 128, 4, 2, 3}, 1, 0.74, 0.74, true, false},
                            {{128, 128, 2, 2, 3}, 2, 0.74, 0.74, false, false},
                            {{192, 128, 4, 2, 3}, 1, 0.69, 0.77, false, true},
                            {{288, 192, 2, 2, 3}, 1, 0.94, 0.94, false, true, true}};
// Fixed cost of the stream-K fix-up (ticket, partial store and reload, the
// extra pipeline ramp of each piece, the idle tail while owners wait), in
// units of one 256x256 k-block; fitted to M = 512 .. 4608 FLUX shapes.
constexpr double kSkFixupBlocks = 11.0;
constexpr int kSkMinIters = 4;

// Time of one k-block of the candidate's tile on a CU, in units of a 256x256
// k-block at full efficiency.
double block_cost(const Cand& c) { return (double)c.t.bm * c.t.bn / 65536.0 / c.eff; }

// A workgroup alone on a CU (fewer tiles than CUs) runs a k-block in
// kLoneBlocks x block_cost: measured on the 128x128 tile at M = 256 .. 1024
// (K = 3072 .. 15360), a lone workgroup takes 0.62 of the time two
// co-resident ones take for a k-block each, not 0.5.
constexpr double kLoneBlocks = 1.1;

// Modelled run time of the busiest CU, in units of one 256x256 k-block.  With
// per_cu workgroups resident on a CU they share it, so a CU's load counts in
// steps of 1/per_cu of a tile.
double dp_time(const Cand& c, int64_t tiles, int64_t kb, int cus) {
  const double partial = tiles < cus ? c.eff / c.eff_partial : 1.0;
  if (c.per_cu > 1 && tiles < cus) return (double)kb * block_cost(c) * kLoneBlocks * partial;
  const int64_t steps = (tiles * c.per_cu + cus - 1) / cus;  // ceil(tiles per CU * per_cu)
  return (double)steps / c.per_cu * (double)kb * block_cost(c) * partial;
}

double sk_time(const Cand& c, int64_t tiles, int64_t kb, int cus, int min_iters) {
  const int64_t P = (int64_t)cus * c.per_cu / kXcds;
  if (P < 1) return 1e300;
  const int64_t tx = (tiles + kXcds - 1) / kXcds;
  const int64_t rounds = tx / P, rem = tx % P;
  const int64_t dp = rem == 0 ? tx : (rounds > 0 ? (rounds - 1) * P : 0);
  const int64_t iters = (tx - dp) * kb;
  const int64_t psk = std::min<int64_t>(P, std::max<int64_t>(1, iters / min_iters));
  const double per = (double)(dp / P) * kb + (double)((iters + psk - 1) / psk);
  return (per * c.per_cu * block_cost(c)) + (iters > 0 ? kSkFixupBlocks : 0.0);
}

// Pick the tile and kernel with the least modelled time.  Tuning overrides
// (convrot_set_tuning): gemm_tile forces the tile, gemm_sk the kernel kind,
// gemm_sk_min the shortest stream-K range.
size_t sk_bytes(const Tile& t, int grid) { return (size_t)kSkPartialOffset + (size_t)grid * t.bm * t.bn * 4; }

Plan choose_plan(int64_t M, int64_t N, int64_t K, bool allow_dma, size_t ws_bytes) {
  const bool allow_sk = allow_dma;
  const int cus = device_cus();
  const int64_t kb = (K + 127) / 128;
  int min_iters = kSkMinIters;
  if (const int v = tuning(kTuneGemmSkMin); v >= 0) min_iters = std::max(1, v);
  int force_sk = -1;
  if (const int v = tuning(kTuneGemmSk); v >= 0) force_sk = v != 0;
  if (!allow_sk) force_sk = 0;

  const Tile* forced = nullptr;
  Tile ft{};
  if (const int v = tuning(kTuneGemmTile); v >= 0) {
    // stages 0: the candidate's own ring depth
    ft = {v & 1023, (v >> 10) & 1023, (v >> 20) & 15, (v >> 24) & 15, (v >> 28) & 7};
    forced = &ft;
  }
  Plan best{{128, 128, 2, 2, 3}, false, 0, min_iters};
  double best_time = 1e300;
  for (const Cand& c : kCands) {
    const bool match = forced && c.t.bm == forced->bm && c.t.bn == forced->bn && c.t.wm == forced->wm &&
                       c.t.wn == forced->wn && (forced->stages == 0 || c.t.stages == forced->stages);
    if ((forced && !match) || (c.dma_only && !allow_dma)) continue;
    const int64_t tiles = ((M + c.t.bm - 1) / c.t.bm) * ((N + c.t.bn - 1) / c.t.bn);
    const double td = dp_time(c, tiles, kb, cus);
    const double ts = sk_time(c, tiles, kb, cus, min_iters);
    const int grid = std::min(kSkMaxGrid, cus * c.per_cu) / kXcds * kXcds;
    const bool sk = !c.no_sk && grid >= kXcds && sk_bytes(c.t, grid) <= ws_bytes &&
                    (force_sk == 1 || (force_sk == -1 && c.sk && ts < td));
    const double tt = sk ? ts : td;
    if (tt < best_time * (1.0 - 1e-9)) {
      best_time = tt;
      best = {c.t, sk, grid, min_iters};
    }
  }
  if (forced && best_time == 1e300) best = {*forced, false, 0, min_iters};  // a tile only the register path has
  return best;
}

// Scratch of convrot_w4a4_gemm_noalloc: a stream-K workspace that is a
// file-scope device array, so that entry point allocates nothing.  Every GPU
// the library runs on holds its own copy (at its own device address) until
// the process ends, and every no-alloc call on that GPU shares it.  Host code
// never names the array itself (on the host it is a stand-in, not a device
// address): it uses the address hipGetSymbolAddress returns for the current
// device, kept in g_noalloc.
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

struct NoAllocState {
  uint8_t* ptr = nullptr;  // device address of `scratch` on this device
  bool cleared = false;    // its control block was zeroed by an eager launch
};
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
NoAllocState g_noalloc[kMaxDevices];

__global__ __launch_bounds__(256) void zero_words_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

int current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return -1;
  return dev;
}

template <int BM, int BN, int WM, int WN, bool APACK, int ODT>
hipError_t launch_tile(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                       int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL((w4a4_gemm_kernel<BM, BN, WM, WN, APACK, ODT>), dim3((unsigned)(tm * tn)), dim3(WM * WN * 64),
                     0, stream, (const uint8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks,
                     tm, tn, gr);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES, int ODT>
hipError_t launch_dma(const Plan& plan, const void* act, const float* xs, const uint8_t* wq, const float* ws,
                      const float* bias, int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr,
                      const Workspace& wsp, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  const int spin = tuning(kTuneSkSpinLimit);
  const SkArgs ska{wsp.ptr, plan.min_iters, spin >= 0 ? spin : kSkSpinLimit};
  const bool sk = plan.sk && wsp.ptr && wsp.bytes >= sk_bytes(plan.t, plan.grid);
  if constexpr (WM * WN == 4 && ((BM == 256 && BN == 256) || (BM == 288 && BN == 192))) {
    if constexpr (BM == 256) {
      if (sk) {
        hipLaunchKernelGGL((w4a4_gemm_agpr_sk_kernel<STAGES, ODT>), dim3((unsigned)plan.grid), dim3(256), 0, stream,
                           (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, tm,
                           tn, ska, gr);
        return hipGetLastError();
      }
      if constexpr (ODT != kF32) {
        // 32x32x32 MFMAs where the grid leaves CUs idle (at most 7/8 of them
        // busy): 5-14 % faster there, 4 % slower with every CU busy, where the
        // shader clock drops further under its higher MFMA rate.  The
        // gemm_mfma32 tuning override forces it off (0) or on (1).
        const int m32 = tuning(kTuneGemmMfma32);
        const bool partial = (int64_t)tm * tn * 8 <= (int64_t)device_cus() * 7;
        if ((m32 == 1 || (m32 < 0 && partial)) && !gr.residual && N % 8 == 0 && M * N * 2 < ((int64_t)1 << 31)) {
          hipLaunchKernelGGL((w4a4_gemm_agpr32_kernel<STAGES, ODT>), dim3((unsigned)(tm * tn)), dim3(256), 0,
                             stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks,
                             kblocks, tm, tn);
          return hipGetLastError();
        }
      }
    }
    if constexpr (ODT != kF32) {
      // More tiles than one round: the persistent kernel (plain epilogue,
      // whole 16-byte output chunks, 32-bit store offsets).  The gemm_persist
      // tuning override turns it off (0) or forces it on a grid of G.
      const int cus = device_cus();
      const int force = tuning(kTuneGemmPersist);
      const bool eligible = !gr.residual && N % 8 == 0 && M * N * 2 < ((int64_t)1 << 31);
      const int64_t tiles = (int64_t)tm * tn;
      int grid = force > 0 ? force : cus;
      grid = std::max(kXcds, grid / kXcds * kXcds);
      if (eligible && force != 0 && (force > 0 || tiles > cus)) {
        grid = (int)std::min<int64_t>(grid, (tiles + kXcds - 1) / kXcds * kXcds);
        const PersistArgs pa{(const int8_t*)act, wq, xs, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks,
                             tm, tn};
        hipLaunchKernelGGL((w4a4_gemm_agpr_persist_kernel<BM, BN, STAGES, ODT>), dim3((unsigned)grid), dim3(256), 0,
                           stream, pa);
        return hipGetLastError();
      }
    }
    hipLaunchKernelGGL((w4a4_gemm_agpr_kernel<BM, BN, STAGES, ODT>), dim3((unsigned)(tm * tn)), dim3(256), 0, stream,
                       (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, tm, tn,
                       gr);
    return hipGetLastError();
  } else {
    // Double-buffered fragments except on the 8-wave 256x256 tile, whose
    // 128-register accumulator leaves no room for a second set.
    constexpr int kPP = (BM == 256 && BN == 256) ? kSingle : kPingPong;
    if (sk) {
      hipLaunchKernelGGL((w4a4_gemm_sk_kernel<BM, BN, WM, WN, kPP, STAGES, ODT>), dim3((unsigned)plan.grid),
                         dim3(WM * WN * 64), 0, stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N,
                         (int)K, nblocks, kblocks, tm, tn, ska, gr);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((w4a4_gemm_dma_kernel<BM, BN, WM, WN, kPP, STAGES, ODT>), dim3((unsigned)(tm * tn)),
                       dim3(WM * WN * 64), 0, stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N,
                       (int)K, nblocks, kblocks, tm, tn, gr);
    return hipGetLastError();
  }
}

template <bool APACK, int ODT>
hipError_t launch_t(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                    int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr, WorkspaceSource src,
                    hipStream_t stream) {
  const bool dma = !APACK && tuning(kTuneGemmNoDma) != 1;
  // The plan with the workspace this call has: none (the entry points without a
  // workspace argument, which allocate nothing) leaves the data-parallel plans,
  // whose outputs are the stream-K plans' bit for bit.
  const Workspace wsp = src.kind == WorkspaceSource::kGiven ? src.given : Workspace{};
  const Plan plan = choose_plan(M, N, K, dma, dma && wsp.ptr ? wsp.bytes : 0);
  const Tile t = plan.t;
  if (dma) {
#define CONVROT_DMA(BM_, BN_, WM_, WN_, S_)                                       \
  if (t.bm == BM_ && t.bn == BN_ && t.wm == WM_ && t.wn == WN_ && t.stages == S_) \
    return launch_dma<BM_, BN_, WM_, WN_, S_, ODT>(plan, act, xs, wq, ws, bias, M, N, K, out, gr, wsp, stream);
    CONVROT_DMA(256, 256, 2, 4, 3)
    CONVROT_DMA(256, 256, 2, 2, 3)
    CONVROT_DMA(256, 128, 4, 2, 3)
    CONVROT_DMA(128, 256, 2, 4, 4)
    CONVROT_DMA(128, 128, 2, 2, 3)
    CONVROT_DMA(192, 128, 4, 2, 3)
    CONVROT_DMA(288, 192, 2, 2, 3)
#undef CONVROT_DMA
  }
#define CONVROT_TILE(BM_, BN_, WM_, WN_)                    \
  if (t.bm == BM_ && t.bn == BN_ && t.wm == WM_ && t.wn == WN_) \
    return launch_tile<BM_, BN_, WM_, WN_, APACK, ODT>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
  CONVROT_TILE(256, 256, 2, 4)
  CONVROT_TILE(256, 256, 4, 2)
  CONVROT_TILE(256, 256, 2, 2)
  CONVROT_TILE(256, 128, 2, 2)
  CONVROT_TILE(256, 128, 4, 2)
  CONVROT_TILE(128, 256, 2, 2)
  CONVROT_TILE(128, 256, 2, 4)
#undef CONVROT_TILE
  return launch_tile<128, 128, 2, 2, APACK, ODT>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
}

template <bool APACK>
hipError_t launch_odt(int odt, const void* act, const float* xs, const uint8_t* wq, const float* ws,
                      const float* bias, int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr,
                      WorkspaceSource src, hipStream_t stream) {
  switch (odt) {
    case kF32: return launch_t<APACK, kF32>(act, xs, wq, ws, bias, M, N, K, out, gr, src, stream);
    case kF16: return launch_t<APACK, kF16>(act, xs, wq, ws, bias, M, N, K, out, gr, src, stream);
    default: return launch_t<APACK, kBF16>(act, xs, wq, ws, bias, M, N, K, out, gr, src, stream);
  }
}

}  // namespace

constexpr int64_t kSmallMMax = 32;
constexpr int64_t kSmallMMaxWide = 64;
constexpr int64_t kSmallMWideElems = 40000000;  // N * K, i.e. 20 MB of int4 weights

namespace {

// Largest M the few-row weight-streaming kernel takes (same results bit for
// bit).  It wins up to M = 32 everywhere measured, and up to 64 while the int4
// weight is at most ~20 MB (beyond that the tiled kernel's 16-17 us floor is
// lower).  The gemm_smallm_max tuning override sets it (0: never).
int64_t smallm_limit(int64_t N, int64_t K) {
  int64_t small_max = N * K <= kSmallMWideElems ? kSmallMMaxWide : kSmallMMax;
  if (const int v = tuning(kTuneGemmSmallmMax); v >= 0) small_max = v;
  return small_max;
}

}  // namespace

hipError_t launch_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                            const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, hipStream_t stream, const GatedResidual& gr,
                            WorkspaceSource src) {
  if (M == 0 || N == 0) return hipSuccess;
  if (act_format == CONVROT_ACT_PACKED)
    return launch_odt<true>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, gr, src, stream);
  if (M <= smallm_limit(N, K))
    return launch_w4a4_smallm((const int8_t*)act, xscales, qweight, wscales, bias, M, N, K, out, out_dtype, stream,
                              gr);
  return launch_odt<false>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, gr, src, stream);
}

bool w4a4_tile_known(int bm, int bn, int wm, int wn, int stages) {
  for (const Cand& c : kCands)
    if (c.t.bm == bm && c.t.bn == bn && c.t.wm == wm && c.t.wn == wn && (stages == 0 || c.t.stages == stages))
      return true;
  // tiles of the register-staged kernel (no LDS ring, so no ring depth)
  constexpr int kRegTiles[][4] = {{256, 256, 2, 4}, {256, 256, 4, 2}, {256, 256, 2, 2}, {256, 128, 2, 2},
                                  {256, 128, 4, 2}, {128, 256, 2, 2}, {128, 256, 2, 4}, {128, 128, 2, 2}};
  for (const auto& t : kRegTiles)
    if (t[0] == bm && t[1] == bn && t[2] == wm && t[3] == wn && stages == 0) return true;
  return false;
}

size_t w4a4_plan_workspace_bytes(int act_format, int64_t M, int64_t N, int64_t K) {
  if (M == 0 || N == 0 || act_format == CONVROT_ACT_PACKED || M <= smallm_limit(N, K)) return 0;
  const bool dma = tuning(kTuneGemmNoDma) != 1;
  const Plan plan = choose_plan(M, N, K, dma, dma ? kSkWorkspaceBytes : 0);
  return plan.sk ? sk_bytes(plan.t, plan.grid) : 0;
}

hipError_t noalloc_scratch(hipStream_t stream, Workspace* out) {
  const int dev = current_device();
  if (dev < 0) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocState& s = g_noalloc[dev];
  if (!s.ptr) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    s.ptr = (uint8_t*)p;
  }
  if (!s.cleared) {
    // The stream-K control block (counters, generations, error word, flags)
    // must start at zero; a fill kernel, stream-ordered before the call's GEMM.
    // Under graph capture the fill becomes part of the graph (harmless: it
    // runs before that graph's GEMM) and the next eager call clears again.
    constexpr int kWords = (int)(kSkPartialOffset / 4);
    hipLaunchKernelGGL(zero_words_kernel, dim3((kWords + 255) / 256), dim3(256), 0, stream, (int*)s.ptr, kWords);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) s.cleared = true;
  }
  *out = {s.ptr, kNoAllocScratchBytes};
  return hipSuccess;
}

int w4a4_workspace_status(const void* workspace, hipStream_t stream, const char** what) {
  *what = nullptr;
  if (hipStreamSynchronize(stream) != hipSuccess) return -1;
  const uint8_t* bufs[2] = {(const uint8_t*)workspace, nullptr};
  if (!workspace) {
    const int dev = current_device();
    if (dev >= 0) {
      std::lock_guard<std::mutex> lock(g_noalloc_mu);
      bufs[1] = g_noalloc[dev].ptr;
    }
  }
  for (const uint8_t* b : bufs) {
    if (!b) continue;
    int err = 0;
    if (hipMemcpy(&err, b + 4 * kSkErrorWord, 4, hipMemcpyDeviceToHost) != hipSuccess) return -1;
    if (err) {
      const int zero = 0;
      if (hipMemcpy((uint8_t*)b + 4 * kSkErrorWord, &zero, 4, hipMemcpyHostToDevice) != hipSuccess) return -1;
      *what = "a stream-K owner gave up waiting for a partial tile (bounded wait); its output tile was written as NaN";
      return 1;
    }
  }
  return 0;
}

// FP6-operand W4A4 GEMM (activation and weight layouts above; K % 128 == 0),
// with the same epilogues as the INT8 kernels.
namespace {

// FP6 tiles and the time per tile each takes relative to a 4-wave 256 x 256
// tile (per tile, at the same K).  The plan takes the tile with the least
// modelled time, rounds of whole tiles over the CUs times the tile's relative
// time.  The 8-wave 256 x 256 tile runs 0.83-0.90 of that time (0.86 in the
// plan), which puts it before 256 x 224 (0.9) wherever both need the same
// rounds: every config-3 shape at 4608 tokens; 128 x 256 fills the CUs at
// a few thousand tokens; 128 x 128 (two workgroups per CU) at 256-1024 tokens
// with N = 3072: 12288 -> 3072 at 512 tokens takes 28.5 us against 42.0 on
// 128 x 256 (its relative time 0.43 measured at 256-1024 tokens); 128 x 192
// (192 tiles: one round) at 1536 tokens, 12288 -> 3072 in 37.0 us against 45.1
// (relative time 0.56 at 1536-2048 tokens).  With eight waves 128 x 256 and
// 128 x 192 run 5-10 % and 2-4 % faster than with four (0.58 and 0.54).
struct Fp6Tile {
  int bm, bn;
  double rel;
};
constexpr Fp6Tile kFp6Tiles[5] = {{256, 256, 0.86}, {256, 224, 0.9}, {128, 256, 0.58}, {128, 128, 0.43}, {128, 192, 0.54}};

Fp6Tile fp6_tile(int64_t M, int64_t N) {
  const int forced = tuning(kTuneFp6Tile);
  if (forced >= 0)
    for (const Fp6Tile& t : kFp6Tiles)
      if ((forced & 1023) == t.bm && (forced >> 10) == t.bn) return t;
  const int64_t cus = device_cus();
  Fp6Tile best = kFp6Tiles[0];
  double best_cost = -1.0;
  for (const Fp6Tile& t : kFp6Tiles) {
    const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
    double cost = (double)((tiles + cus - 1) / cus) * t.rel;
    // Two 128 x 128 workgroups share a CU and the dispatcher refills CUs as
    // workgroups finish, so a grid of many such tiles runs in time nearly
    // linear in the tile count (0.33 per CU-load of tiles from two full
    // rounds of two a CU on: 1536 x 3072 -> 12288, 1152 tiles, 40.8 us
    // against 44.5 on 128 x 192); fewer tiles keep the rounded model.
    if (t.bm == 128 && t.bn == 128 && tiles >= 4 * cus) cost = (double)tiles / (double)cus * 0.33;
    if (best_cost < 0 || cost < best_cost - 1e-9) {
      best = t;
      best_cost = cost;
    }
  }
  return best;
}

template <int BM, int BN, int ODT, bool CW>
hipError_t launch_fp6_tile(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                           const float* bias, int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr,
                           hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  // 8 waves on 256 x 256, 128 x 256 and 128 x 192; 4 on 256 x 224 and 128 x 128
  constexpr int WN = ((BM == 256 && BN == 256) || (BM == 128 && BN >= 192)) ? 4 : 2;
  hipLaunchKernelGGL((w4a4_gemm_fp6_kernel<BM, BN, ODT, CW, WN>), dim3((unsigned)(tm * tn)), dim3(WN * 128), 0, stream, act6,
                     xscales, w6, wscales, bias, out, (int)M, (int)N, (int)K, nblocks, tm, tn, gr);
  return hipGetLastError();
}

template <int ODT, bool CW>
hipError_t launch_fp6_t(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                        const float* bias, int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr,
                        hipStream_t stream) {
  const Fp6Tile t = fp6_tile(M, N);
  if (t.bm == 256 && t.bn == 224)
    return launch_fp6_tile<256, 224, ODT, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
  if (t.bm == 128 && t.bn == 128)
    return launch_fp6_tile<128, 128, ODT, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
  if (t.bm == 128 && t.bn == 192)
    return launch_fp6_tile<128, 192, ODT, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
  if (t.bm == 128)
    return launch_fp6_tile<128, 256, ODT, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
  return launch_fp6_tile<256, 256, ODT, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
}

template <bool CW>
hipError_t launch_fp6_odt(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                          const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                          hipStream_t stream, const GatedResidual& gr) {
  switch (out_dtype) {
    case kF32: return launch_fp6_t<kF32, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
    case kF16: return launch_fp6_t<kF16, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
    default: return launch_fp6_t<kBF16, CW>(act6, xscales, w6, wscales, bias, M, N, K, out, gr, stream);
  }
}

}  // namespace

bool fp6_tile_known(int bm, int bn) {
  for (const Fp6Tile& t : kFp6Tiles)
    if (t.bm == bm && t.bn == bn) return true;
  return false;
}

void fp6_plan_tile(int64_t M, int64_t N, int* bm, int* bn) {
  const Fp6Tile t = fp6_tile(M, N);
  *bm = t.bm;
  *bn = t.bn;
}

hipError_t launch_w4a4_gemm_fp6(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                                const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                                hipStream_t stream, const GatedResidual& gr, bool compact_weights) {
  if (M == 0 || N == 0) return hipSuccess;
  if (compact_weights)
    return launch_fp6_odt<true>(act6, xscales, w6, wscales, bias, M, N, K, out, out_dtype, stream, gr);
  return launch_fp6_odt<false>(act6, xscales, w6, wscales, bias, M, N, K, out, out_dtype, stream, gr);
}

}  // namespace convrot
