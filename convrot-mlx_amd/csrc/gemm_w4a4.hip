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
template <int ODT, int TM, int TN, int SHIFT, bool LDS_OPS = false>
__device__ __forceinline__ void epilogue(const i32x4 (&acc)[TN / 16][TM / 16], uint8_t* region, int lane,
                                         int mw, int nw, int M, int N, const float* __restrict__ xscales,
                                         const float* __restrict__ wscales, const float* __restrict__ bias,
                                         void* __restrict__ out, const GatedResidual& gr, int m0 = 0,
                                         int n0 = 0) {
  constexpr int FM = TM / 16, FN = TN / 16;
  float xs[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = mw + fm * 16 + (lane & 15);
    if constexpr (LDS_OPS) xs[fm] = xscales[m - m0];
    else xs[fm] = xscales[m < M ? m : M - 1];
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
        for (int r = 0; r < 4; ++r) o[r] = (((float)(acc[fn][fm][r] >> SHIFT) * xs[fm]) * wsv[r]) + bv[r];
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
        for (int r = 0; r < 4; ++r) o[r] = (((float)(acc[fn][fm][r] >> SHIFT) * xs[fm]) * wsv[r]) + bv[r];
        const uint2 w = ODT == kBF16 ? make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]))
                                     : make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
        *(uint2*)(region + (fm * 16 + (lane & 15)) * RS + nl * 2) = w;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int CPR = TN / 8;        // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;      // rows per wave instruction
    constexpr int NIT = TM / RPI;      // write-back iterations
    const int cr = lane / CPR, cc = lane % CPR;
    const int n = nw + cc * 8;
    const bool vec = (N & 7) == 0 && n + 8 <= N;
    auto store_row = [&](int it, uint4 v) {
      uint16_t* dst = (uint16_t*)out + (int64_t)(mw + it * RPI + cr) * N + n;
      if (vec) {
        *(uint4*)dst = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (n + j < N) dst[j] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
      }
    };
    if (!gr.residual) {
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int rl = it * RPI + cr;
        if (mw + rl >= M || n >= N) continue;
        store_row(it, *(const uint4*)(region + rl * RS + cc * 16));
      }
    } else {
      // Residual and gate loads of BATCH rows go out before their stores (a
      // load cannot be moved above a store that may alias it, so one row at a
      // time would wait a memory round trip per row).
      constexpr int BATCH = NIT < 8 ? NIT : 8;
      static_assert(NIT % BATCH == 0, "write-back batches");
#pragma unroll
      for (int b0 = 0; b0 < NIT; b0 += BATCH) {
        Gated8 ops[BATCH];
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const int m = mw + (b0 + i) * RPI + cr;
          if (m < M && n < N) gate_load8<ODT>(gr, m, n, N, vec, ops[i]);
        }
#pragma unroll
        for (int i = 0; i < BATCH; ++i) {
          const int rl = (b0 + i) * RPI + cr;
          if (mw + rl >= M || n >= N) continue;
          store_row(b0 + i, gate_apply8<ODT>(ops[i], *(const uint4*)(region + rl * RS + cc * 16)));
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
//  kPingPong two full sets, block i+1 read during block i's MFMAs.
// (A 4-wave 256x256 tile with one wave per SIMD and the accumulator in the
// AGPRs, fed by k-step-split reads, measured 1.8x slower: the compiler cannot
// keep a 256-register accumulator in place and spills inside the loop.)
enum Pipe : int { kSingle = 0, kPingPong = 1 };

template <int BM, int BN, int WM, int WN, int PIPE, int STAGES = 3>
struct DmaEngine {
  static constexpr int NW = WM * WN;
  static constexpr int TM = BM / WM, TN = BN / WN;
  static constexpr int FM = TM / 16, FN = TN / 16;
  static constexpr int A_FRAGS = (BM / 16) * 2, B_FRAGS = BN / 16;
  static constexpr int LOADS = A_FRAGS + B_FRAGS;
  static constexpr int STAGE_BYTES = LOADS * 1024;
  // Epilogue operands of the tile, loaded into LDS with the first k-blocks:
  // xs[m0 .. m0+255], ws[n0 .. n0+255], bias[n0 .. n0+255] (1 KB each).
  static constexpr int EPI_OFF = STAGES * STAGE_BYTES;
  static constexpr int EPI_BYTES = 3 * 1024;
  static constexpr int EPI_DMAS = 3 * 4;  // 256-byte dword DMAs
  static constexpr int SMEM_BYTES = EPI_OFF + EPI_BYTES;
  static constexpr int LPW = LOADS / NW;  // DMA instructions per wave per k-block
  static constexpr int APW = A_FRAGS / NW, BPW = B_FRAGS / NW;  // of which activation / weight
  static constexpr int SHIFT = 4;         // weights unpacked x16: acc = 16 * dot
  static constexpr int STAGING = TM * (TN * 2 + 16);  // epilogue LDS bytes per wave
  static_assert(LOADS % NW == 0, "fragment loads must split evenly over waves");
  static_assert(A_FRAGS % NW == 0 && B_FRAGS % NW == 0, "each wave loads APW + BPW pieces");
  static_assert(NW * STAGING <= EPI_OFF, "epilogue staging exceeds the ring");
  static_assert(BM <= 256 && BN <= 256, "one KB of LDS per epilogue operand");
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
  __device__ __forceinline__ const float* epi_xs() const { return (const float*)(smem + EPI_OFF); }
  __device__ __forceinline__ const float* epi_ws() const { return (const float*)(smem + EPI_OFF + 1024); }
  __device__ __forceinline__ const float* epi_bias() const { return (const float*)(smem + EPI_OFF + 2048); }

  // Load the tile's epilogue operands into LDS: 12 dword DMAs of 256 bytes,
  // DMA d by wave d % NW.  Entries past M or N, and all of a missing
  // bias, read as zero.  Issued before the run's prologue: vmcnt retires in
  // issue order, so the run's first DMA wait also retires these, and the
  // barrier after the run publishes them to every wave.  The area must not be
  // read by a previous epilogue when they are issued.
  __device__ __forceinline__ void issue_epi(const float* xscales, const float* wscales, const float* bias, int M,
                                            int N, int m0, int n0) {
    for (int d = wave; d < EPI_DMAS; d += NW) {  // array d / 4, quarter d % 4
      const int arr = d >> 2;
      const float* base = arr == 0 ? xscales + m0 : arr == 1 ? wscales + n0 : (bias ? bias + n0 : wscales);
      const int count = arr == 0 ? M - m0 : (arr == 1 || bias) ? N - n0 : 0;
      const i32x4_sgpr r = buffer_rsrc(base, (uint32_t)count * 4u);
      dma4(r, (uint32_t)((d & 3) * 256 + lane * 4), smem_addr + (uint32_t)(EPI_OFF + arr * 1024 + (d & 3) * 256));
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
    body(kb0, n, acc, nullptr);
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
    constexpr int AHEAD = PIPE == kPingPong ? STAGES : STAGES - 1;
#pragma unroll
    for (int s = 0; s < AHEAD; ++s)
      if (s < n) issue(kb0 + s, s);
  }

  // The rest of a run after prologue(kb0, n).  The prologue's DMAs must be the
  // newest vector-memory operations of the wave.  vmcnt retires in issue
  // order, so the first wait also retires everything the wave issued before
  // the prologue; if `flag` is set, lane 0 raises it right after that wait.
  __device__ __forceinline__ void body(int kb0, int n, i32x4 (&acc)[FN][FM], int* flag) {
    auto raise = [&]() {
      if (flag && lane == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// ---- stream-K
//
// Workspace (device memory owned by the launcher, one per device and stream):
//   int32 word 32 g          ticket counter of workgroup group g (one group per XCD)
//   int32 word 256 + 32 g    finished-workgroup counter of group g
//   int32 words [512, 512+G*NW) partial-ready flag of each (workgroup slot, wave)
//   bytes [kSkPartialOffset, ...)  one int32 partial tile per workgroup slot
// Each counter has a 128-byte line to itself: every workgroup of the launch
// performs two device-scope atomics on its group's counters, and atomics on
// one line are serialized.
// Every counter and flag is back at zero when a launch ends, so consecutive
// launches on one stream share the workspace; launches that overlap in time
// (two streams) must not.
constexpr int kSkLineWords = 32;
constexpr int kSkDoneWord = kXcds * kSkLineWords;
constexpr int kSkCtlWords = 2 * kSkDoneWord;
constexpr int64_t kSkPartialOffset = 32768;
constexpr int kSkMaxGrid = 512;  // <= 64 workgroups per group: one lane per contributor when polling
constexpr int kSkMaxWaves = 8;
static_assert(kSkCtlWords + kSkMaxGrid * kSkMaxWaves <= kSkPartialOffset / 4, "flags overflow the control block");
constexpr int kSkSpinLimit = 1 << 22;  // ~1 s of s_sleep: a lost flag ends the wait instead of hanging

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
template <int OFF>
__device__ __forceinline__ i32x4 load_dev16(const void* p) {
  i32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off offset:%2 sc1" : "=v"(v) : "v"(p), "i"(OFF) : "memory");
  return v;
}

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
// (8 beside a 32-fragment accumulator), one wait per batch.
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

// Lane i < n waits for flag first[i * stride] (all in parallel), then clears it.
__device__ __forceinline__ void sk_wait_flags(int* first, int stride, int n, int lane) {
  int* f = first + (int64_t)lane * stride;
  bool seen = lane >= n;
  for (int it = 0; it < kSkSpinLimit; ++it) {
    if (!seen) seen = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
    if (__ballot(!seen) == 0) break;
    __builtin_amdgcn_s_sleep(4);
  }
  if (lane < n) __hip_atomic_store(f, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Persistent stream-K GEMM (Osama et al., "Stream-K: Work-centric Parallel
// Decomposition for Dense Matrix-Matrix Multiplication on the GPU", 2023), in
// its data-parallel + stream-K hybrid form, run per XCD.
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
// tickets themselves, so the kernel finishes whatever the residency.
template <int BM, int BN, int WM, int WN, int PIPE, int STAGES, int ODT>
__global__ __launch_bounds__(WM* WN * 64) void w4a4_gemm_sk_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n, uint8_t* __restrict__ work, int min_iters,
    GatedResidual gr) {
  using E = DmaEngine<BM, BN, WM, WN, PIPE, STAGES>;
  constexpr int FN = E::FN, FM = E::FM, NW = E::NW;
  static_assert(NW <= kSkMaxWaves, "flag block sized for 8 waves");
  __shared__ __attribute__((aligned(1024))) uint8_t smem[E::SMEM_BYTES];
  __shared__ int s_ticket;

  int* ctl = (int*)work;
  int* flags = ctl + kSkCtlWords;
  uint8_t* partials = work + kSkPartialOffset;
  const int group = blockIdx.x % kXcds;
  const int P = gridDim.x / kXcds;
  if (threadIdx.x == 0) s_ticket = atomicAdd(&ctl[group * kSkLineWords], 1);
  __syncthreads();
  const int p = __builtin_amdgcn_readfirstlane(s_ticket);
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
  const int psk = min(P, max(1, sk_iters / max(1, min_iters)));
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
    e.body(k0, k1 - k0, acc, pending);
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
        if (e.lane == 0) __hip_atomic_store(flag, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      if (k0 > 0) {
        // Lower tickets qf .. p-1 hold the tile's earlier k-blocks; ticket q's
        // range starts at sk_iters * q / psk.
        const int tstart = (t - dp) * kblocks;
        int qf = p - 1;
        while (sk_iters * qf / psk > tstart) --qf;
        sk_wait_flags(&flags[(group * P + qf) * NW + e.wave], NW, p - qf, e.lane);
        for (int q = qf; q < p; ++q)
          sk_add_partial<FN, FM>(partials + (int64_t)(group * P + q) * (BM * BN * 4) + wave_off, e.lane, acc);
      }
      __syncthreads();  // ring -> epilogue staging
      epilogue<ODT, E::TM, E::TN, E::SHIFT, true>(acc, e.staging(), e.lane, m0 + e.wm * E::TM, n0 + e.wn * E::TN,
                                                  M, N, e.epi_xs(), e.epi_ws(), e.epi_bias(), out, gr, m0, n0);
      __syncthreads();  // staging -> next item's DMA
    }
    t = nt;
    k0 = nk0;
    k1 = nk1;
    have = more;
  }

  // The last workgroup of the group to finish rearms the ticket counters.
  if (threadIdx.x == 0) {
    if (atomicAdd(&ctl[kSkDoneWord + group * kSkLineWords], 1) == P - 1) {
      __hip_atomic_store(&ctl[group * kSkLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&ctl[kSkDoneWord + group * kSkLineWords], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
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
// state on MI355X (256x256 moves half the L2 bytes per MFMA of 128x128 but
// runs one workgroup per CU; 128x128 fits two per CU).  `sk` marks the tiles
// the stream-K kernel runs well: the 256x256 one spills registers there and
// 128x128 pieces are too short.
//
// The 192x128 tile moves more L2 bytes per MFMA than the 256x256 one and
// sustains 0.75 of its rate with every CU busy, but 0.83 when its grid is a
// single round that leaves CUs idle (1536 tokens: 192 tiles at N = 3072,
// 21.2 us against 24.2-25.4 us for every other tile).
struct Cand {
  Tile t;
  int per_cu;
  double eff;
  double eff_partial;  // eff when the grid is one round of fewer tiles than CUs
  bool sk;
  bool dma_only;  // no register-staged (packed-activation) variant
};
constexpr Cand kCands[5] = {{{256, 256, 2, 4, 3}, 1, 1.0, 1.0, false, false},
                            {{128, 256, 2, 4, 4}, 1, 0.85, 0.85, true, false},
                            {{256, 128, 4, 2, 3}, 1, 0.8, 0.8, true, false},
                            {{128, 128, 2, 2, 3}, 2, 0.8, 0.8, false, false},
                            {{192, 128, 4, 2, 3}, 1, 0.75, 0.83, false, true}};
// Fixed cost of the stream-K fix-up (ticket, partial store and reload, the
// extra pipeline ramp of each piece, the idle tail while owners wait), in
// units of one 256x256 k-block; fitted to M = 512 .. 4608 FLUX shapes.
constexpr double kSkFixupBlocks = 10.0;
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

// Pick the tile and kernel with the least modelled time.  Overrides for
// tuning sweeps and tests: CONVROT_GEMM_TILE=BMxBN[wWMxWN[sS]] forces the tile,
// CONVROT_GEMM_SK=0|1 forces the kernel kind, CONVROT_GEMM_SK_MIN sets the
// shortest stream-K range.
Plan choose_plan(int64_t M, int64_t N, int64_t K, bool allow_sk) {
  const int cus = device_cus();
  const int64_t kb = (K + 127) / 128;
  int min_iters = kSkMinIters;
  if (const char* env = getenv("CONVROT_GEMM_SK_MIN")) min_iters = std::max(1, atoi(env));
  int force_sk = -1;
  if (const char* env = getenv("CONVROT_GEMM_SK")) force_sk = atoi(env) != 0;
  if (!allow_sk) force_sk = 0;

  const Tile* forced = nullptr;
  Tile ft{};
  if (const char* env = getenv("CONVROT_GEMM_TILE")) {
    int bm = 0, bn = 0, wm = 2, wn = 2, stages = 0;  // 0: the candidate's own ring depth
    if (sscanf(env, "%dx%dw%dx%ds%d", &bm, &bn, &wm, &wn, &stages) >= 2) {
      ft = {bm, bn, wm, wn, stages};
      forced = &ft;
    }
  }
  Plan best{{128, 128, 2, 2, 3}, false, 0, min_iters};
  double best_time = 1e300;
  for (const Cand& c : kCands) {
    const bool match = forced && c.t.bm == forced->bm && c.t.bn == forced->bn && c.t.wm == forced->wm &&
                       c.t.wn == forced->wn && (forced->stages == 0 || c.t.stages == forced->stages);
    if ((forced && !match) || (c.dma_only && !allow_sk)) continue;
    const int64_t tiles = ((M + c.t.bm - 1) / c.t.bm) * ((N + c.t.bn - 1) / c.t.bn);
    const double td = dp_time(c, tiles, kb, cus);
    const double ts = sk_time(c, tiles, kb, cus, min_iters);
    const int grid = std::min(kSkMaxGrid, cus * c.per_cu) / kXcds * kXcds;
    const bool sk = grid >= kXcds && (force_sk == 1 || (force_sk == -1 && c.sk && ts < td));
    const double tt = sk ? ts : td;
    if (tt < best_time * (1.0 - 1e-9)) {
      best_time = tt;
      best = {c.t, sk, grid, min_iters};
    }
  }
  if (forced && best_time == 1e300) best = {*forced, false, 0, min_iters};  // a tile only the register path has
  return best;
}

// Stream-K workspace, one per (device, stream): launches on one stream are
// ordered and leave the control words zeroed, so they share it.  It is the
// library's only allocation (32 MiB for the 8-wave tiles on 256 CUs), made on
// the first stream-K launch of a stream and kept for the process;
// CONVROT_GEMM_SK=0 keeps every launch data-parallel and allocation-free.
struct SkBuffer {
  int dev;
  hipStream_t stream;
  uint8_t* ptr;
  size_t bytes;
};
std::mutex g_sk_mu;
std::vector<SkBuffer> g_sk_buffers;

// Returns nullptr (and the caller runs the data-parallel kernel) when the
// buffer cannot be made: allocation failure, or a stream under graph capture
// that has no buffer yet.
uint8_t* sk_workspace(hipStream_t stream, size_t bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_sk_mu);
  SkBuffer* slot = nullptr;
  for (SkBuffer& b : g_sk_buffers)
    if (b.dev == dev && b.stream == stream) slot = &b;
  if (slot && slot->bytes >= bytes) return slot->ptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return nullptr;
  if (slot) {  // grow: earlier launches on this stream may still use the old buffer
    if (hipStreamSynchronize(stream) != hipSuccess) return nullptr;
    (void)hipFree(slot->ptr);
    slot->ptr = nullptr;
    slot->bytes = 0;
  } else {
    g_sk_buffers.push_back({dev, stream, nullptr, 0});
    slot = &g_sk_buffers.back();
  }
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (hipMemsetAsync(p, 0, (size_t)kSkPartialOffset, stream) != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) {
    (void)hipFree(p);
    return nullptr;
  }
  slot->ptr = (uint8_t*)p;
  slot->bytes = bytes;
  return slot->ptr;
}

// Bytes a stream-K launch of the plan needs: the control block plus one int32
// partial tile per workgroup.  The buffer of a (device, stream) only grows.
size_t sk_workspace_bytes(const Plan& plan) {
  return (size_t)kSkPartialOffset + (size_t)plan.grid * (size_t)plan.t.bm * (size_t)plan.t.bn * 4;
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
                      hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  // Double-buffered fragments except on the 8-wave 256x256 tile, whose
  // 128-register accumulator leaves no room for a second set.
  constexpr int kPP = (BM == 256 && BN == 256) ? kSingle : kPingPong;
  if (plan.sk) {
    if (uint8_t* work = sk_workspace(stream, sk_workspace_bytes(plan))) {
      hipLaunchKernelGGL((w4a4_gemm_sk_kernel<BM, BN, WM, WN, kPP, STAGES, ODT>), dim3((unsigned)plan.grid),
                         dim3(WM * WN * 64), 0, stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N,
                         (int)K, nblocks, kblocks, tm, tn, work, plan.min_iters, gr);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((w4a4_gemm_dma_kernel<BM, BN, WM, WN, kPP, STAGES, ODT>), dim3((unsigned)(tm * tn)), dim3(WM * WN * 64),
                     0, stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks,
                     tm, tn, gr);
  return hipGetLastError();
}

template <bool APACK, int ODT>
hipError_t launch_t(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                    int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const bool dma = !APACK && !getenv("CONVROT_GEMM_NO_DMA");
  const Plan plan = choose_plan(M, N, K, dma);
  const Tile t = plan.t;
  if (dma) {
#define CONVROT_DMA(BM_, BN_, WM_, WN_, S_)                                       \
  if (t.bm == BM_ && t.bn == BN_ && t.wm == WM_ && t.wn == WN_ && t.stages == S_) \
    return launch_dma<BM_, BN_, WM_, WN_, S_, ODT>(plan, act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    CONVROT_DMA(256, 256, 2, 4, 3)
    CONVROT_DMA(256, 128, 4, 2, 3)
    CONVROT_DMA(128, 256, 2, 4, 4)
    CONVROT_DMA(128, 128, 2, 2, 3)
    CONVROT_DMA(192, 128, 4, 2, 3)
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
                      hipStream_t stream) {
  switch (odt) {
    case kF32: return launch_t<APACK, kF32>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    case kF16: return launch_t<APACK, kF16>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    default: return launch_t<APACK, kBF16>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
  }
}

}  // namespace

constexpr int64_t kSmallMMax = 32;
constexpr int64_t kSmallMMaxWide = 64;
constexpr int64_t kSmallMWideElems = 40000000;  // N * K, i.e. 20 MB of int4 weights

hipError_t launch_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                            const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, hipStream_t stream, const GatedResidual& gr) {
  if (M == 0 || N == 0) return hipSuccess;
  if (act_format == CONVROT_ACT_PACKED)
    return launch_odt<true>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, gr, stream);
  // Few rows: the weight-streaming kernel (same results bit for bit).  It
  // wins up to M = 32 everywhere measured, and up to 64 while the int4 weight
  // is at most ~20 MB (beyond that the tiled kernel's 16-17 us floor is lower).
  // CONVROT_GEMM_SMALLM_MAX sets the largest M it takes (0: never).
  int64_t small_max = N * K <= kSmallMWideElems ? kSmallMMaxWide : kSmallMMax;
  if (const char* env = getenv("CONVROT_GEMM_SMALLM_MAX")) small_max = atoll(env);
  if (M <= small_max)
    return launch_w4a4_smallm((const int8_t*)act, xscales, qweight, wscales, bias, M, N, K, out, out_dtype, stream,
                              gr);
  return launch_odt<false>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, gr, stream);
}

}  // namespace convrot
