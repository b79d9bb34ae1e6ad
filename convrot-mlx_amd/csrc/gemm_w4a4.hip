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
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n) {
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


typedef int i32x4_sgpr __attribute__((ext_vector_type(4)));

// Raw buffer resource (stride 0): accesses at or beyond `bytes` read as zero.
// Built from wave-uniform values so it lives in SGPRs.
__device__ __forceinline__ i32x4_sgpr buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  return (i32x4_sgpr){__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                      __builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32)),
                      __builtin_amdgcn_readfirstlane((int)bytes), 0x00020000};
}

// One wave-wide 16-byte-per-lane load from a buffer straight into LDS at
// lds_addr + 16 * lane (buffer_load_dwordx4 ... lds, address in M0).  Issued
// through asm so the compiler does not add conservative vmcnt waits before
// LDS reads; the kernel orders these loads with explicit waits + barriers.
__device__ __forceinline__ void dma16(i32x4_sgpr rsrc, uint32_t voffset, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc), "{m0}"(lds_addr) : "memory");
}

// s_waitcnt on vmcnt only (expcnt and lgkmcnt left at "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  asm volatile("" ::: "memory");
}

// Fused epilogue of one wave's TM x TN accumulator tile:
//   out = dtype(((float(acc >> SHIFT) * xs[m]) * ws[n]) + bias[n])   (core.py:1168-1171)
// 16-bit outputs are staged through the wave's LDS region (row stride TN*2+16
// bytes) and written back as 16-byte stores covering whole row segments; the
// MFMA accumulator layout (4 consecutive n of one m per lane) would otherwise
// produce 32-byte write fragments.  float32 outputs store 4 values per lane.
template <int ODT, int TM, int TN, int SHIFT>
__device__ __forceinline__ void epilogue(const i32x4 (&acc)[TN / 16][TM / 16], uint8_t* region, int lane,
                                         int mw, int nw, int M, int N, const float* __restrict__ xscales,
                                         const float* __restrict__ wscales, const float* __restrict__ bias,
                                         void* __restrict__ out) {
  constexpr int FM = TM / 16, FN = TN / 16;
  float xs[FM];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = mw + fm * 16 + (lane & 15);
    xs[fm] = xscales[m < M ? m : M - 1];
  }
  if constexpr (ODT == kF32) {
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int n = nw + fn * 16 + 4 * (lane >> 4);
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
        const int m = mw + fm * 16 + (lane & 15);
        if (m >= M) continue;
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = (((float)(acc[fn][fm][r] >> SHIFT) * xs[fm]) * wsv[r]) + bv[r];
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
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nn = min(nw + nl + r, N - 1);
        wsv[r] = wscales[nn];
        bv[r] = bias ? bias[nn] : 0.0f;
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
    const int cr = lane / CPR, cc = lane % CPR;
    const bool vec_ok = (N & 7) == 0;
#pragma unroll
    for (int r0 = 0; r0 < TM; r0 += RPI) {
      const int rl = r0 + cr;
      const int m = mw + rl, n = nw + cc * 8;
      if (m >= M || n >= N) continue;
      const uint4 v = *(const uint4*)(region + rl * RS + cc * 16);
      uint16_t* dst = (uint16_t*)out + (int64_t)m * N + n;
      if (vec_ok && n + 8 <= N) {
        *(uint4*)dst = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (n + j < N) dst[j] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
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
// a STAGES-deep LDS ring, so no registers stage the data and loads run
// STAGES-1 blocks ahead of the MFMAs.  Every activation load reads whole
// 128-byte lines; inside LDS the 16-byte chunks of each row are permuted by
// a_swizzle so that the MFMA fragment reads (16 rows x 16 bytes) are
// bank-conflict free.  Out-of-range rows/blocks read as zero through the
// buffer range check (no branches in the loop).
template <int BM, int BN, int WM, int WN, int STAGES, bool PINGPONG, int ODT>
__global__ __launch_bounds__(WM* WN * 64) void w4a4_gemm_dma_kernel(
    const int8_t* __restrict__ act, const float* __restrict__ xscales, const uint8_t* __restrict__ wq,
    const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out, int M, int N,
    int K, int nblocks, int kblocks, int tiles_m, int tiles_n) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  constexpr int A_FRAGS = (BM / 16) * 2, B_FRAGS = BN / 16;
  constexpr int LOADS = A_FRAGS + B_FRAGS;
  constexpr int STAGE_BYTES = LOADS * 1024;
  static_assert(LOADS % NW == 0, "fragment loads must split evenly over waves");
  constexpr int LPW = LOADS / NW;
  constexpr int SHIFT = 4;  // weights unpacked x16

  __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;

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

  const int rows_valid = min(BM, M - m0);
  const i32x4_sgpr ra = buffer_rsrc(act + (int64_t)m0 * K, (uint32_t)rows_valid * (uint32_t)K);
  const uint8_t* wbase = wq + (int64_t)(n0 / 16) * 1024;
  const uint32_t wbytes = (uint32_t)(((int64_t)kblocks * nblocks - n0 / 16) * 1024);
  const i32x4_sgpr rw = buffer_rsrc(wbase, wbytes);
  const uint32_t smem_addr = (uint32_t)(uintptr_t)smem;

  // This wave's fragment loads: resource, per-lane byte offset at k-block 0
  // and byte stride per k-block (selected once, branch-free in the loop).
  i32x4_sgpr rs[LPW];
  uint32_t voff[LPW], kstride[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int j = wave * LPW + i;
    const bool is_a = j < A_FRAGS;
    // A: instruction j covers rows 8j .. 8j+7 of the tile, 128 bytes each (full
    // cache lines).  LDS slot p of row r holds 16-byte chunk p ^ swz(r).
    const int r = 8 * j + (lane >> 3);
    const int chunk = (lane & 7) ^ a_swizzle(r);
    const uint32_t va = (uint32_t)(r * K + 16 * chunk);
    const uint32_t vb = (uint32_t)((j - A_FRAGS) * 1024 + lane * 16);
    voff[i] = is_a ? va : vb;
    kstride[i] = is_a ? 128u : (uint32_t)nblocks * 1024u;
#pragma unroll
    for (int c = 0; c < 4; ++c) rs[i][c] = is_a ? ra[c] : rw[c];
  }
  auto issue = [&](int kb, int stage) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const uint32_t dst = smem_addr + (uint32_t)(stage * STAGE_BYTES + (wave * LPW + i) * 1024);
      dma16(rs[i], voff[i] + (uint32_t)kb * kstride[i], dst);
    }
  };

  i32x4 acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};

  // Fragments of one k-block held in registers: packed weights (both k-steps)
  // and int8 activations for k-steps 0 and 1.
  struct Frags {
    uint4 b[FN];
    i32x4 a[2][FM];
  };
  auto read_frags = [&](int stage, Frags& f) {
    const uint8_t* st = smem + stage * STAGE_BYTES;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) f.b[fn] = *(const uint4*)(st + (A_FRAGS + wn * FN + fn) * 1024 + lane * 16);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        // row m of 16-row group g, features 32q + 16ks .. +16 = chunk 2q + ks
        const int row = (wm * FM + fm) * 16 + (lane & 15);
        const int chunk = (2 * (lane >> 4) + ks) ^ a_swizzle(row);
        f.a[ks][fm] = *(const i32x4*)(st + row * 128 + chunk * 16);
      }
  };
  auto mma = [&](const Frags& f) {
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
  };

  // Pipeline: DMA runs STAGES-1 blocks ahead; fragments of block kb+1 are
  // read from LDS into the spare register set while block kb's MFMAs run.
  // One barrier per block: it publishes DMA(kb+1) and retires all reads of
  // stage kb % STAGES, which the next DMA then refills.
  static_assert(STAGES == 3, "pipeline written for three LDS stages");
  Frags f0;
  [[maybe_unused]] Frags f1;
  if constexpr (PINGPONG) {
    // DMA three blocks ahead; block kb+1's fragments are read into the spare
    // register set while block kb's MFMAs run.  The barrier of step kb
    // publishes DMA(kb+1) and retires every wave's reads of stage kb % 3
    // (issued in step kb-1), which DMA(kb+3) then refills.
#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue(s, s);
    wait_vmcnt<2 * LPW>();
    __syncthreads();
    read_frags(0, f0);
    auto step = [&](int kb, Frags& cur, Frags& nxt) {
      wait_vmcnt<LPW>();
      __syncthreads();
      issue(kb + STAGES, kb % STAGES);
      if (kb + 1 < kblocks) read_frags((kb + 1) % STAGES, nxt);
      mma(cur);
    };
    int kb = 0;
    for (; kb + 1 < kblocks; kb += 2) {
      step(kb, f0, f1);
      step(kb + 1, f1, f0);
    }
    if (kb < kblocks) step(kb, f0, f1);
  } else {
    // One register set: DMA two blocks ahead.  The barrier of iteration kb
    // publishes DMA(kb) and retires every wave's reads of stage (kb-1) % 3,
    // which DMA(kb+2) then refills.
    issue(0, 0);
    issue(1, 1);
    for (int kb = 0; kb < kblocks; ++kb) {
      wait_vmcnt<LPW>();
      __syncthreads();
      issue(kb + 2, (kb + 2) % STAGES);
      read_frags(kb % STAGES, f0);
      mma(f0);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();  // all waves done with the LDS ring before it is reused for output staging
  static_assert(NW * TM * (TN * 2 + 16) <= STAGES * STAGE_BYTES, "epilogue staging exceeds LDS");
  epilogue<ODT, TM, TN, SHIFT>(acc, smem + wave * TM * (TN * 2 + 16), lane, m0 + wm * TM, n0 + wn * TN, M, N,
                               xscales, wscales, bias, out);
}

struct Tile {
  int bm, bn, wm, wn;
};

template <int BM, int BN, int WM, int WN, bool APACK, int ODT>
hipError_t launch_tile(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                       int64_t M, int64_t N, int64_t K, void* out, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL((w4a4_gemm_kernel<BM, BN, WM, WN, APACK, ODT>), dim3((unsigned)(tm * tn)), dim3(WM * WN * 64),
                     0, stream, (const uint8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks,
                     tm, tn);
  return hipGetLastError();
}

// Tile choice: maximise (busy fraction of the last round of workgroups) x
// (measured per-tile efficiency of the tile).  256x256 moves half the L2 bytes
// per MFMA of 128x128 but runs one workgroup per CU; 128x128 fits two per CU.
// CONVROT_GEMM_TILE=BMxBN[wWMxWN] overrides (tuning sweeps).
Tile choose_tile(int64_t M, int64_t N) {
  if (const char* env = getenv("CONVROT_GEMM_TILE")) {
    int bm = 0, bn = 0, wm = 2, wn = 2;
    if (sscanf(env, "%dx%dw%dx%d", &bm, &bn, &wm, &wn) >= 2) return {bm, bn, wm, wn};
  }
  struct Cand {
    Tile t;
    int per_cu;
    double eff;
  };
  const Cand cands[4] = {{{256, 256, 2, 4}, 1, 1.0}, {{128, 256, 2, 4}, 1, 0.85}, {{256, 128, 4, 2}, 1, 0.8},
                         {{128, 128, 2, 2}, 2, 0.8}};
  Tile best = {128, 128, 2, 2};
  double best_score = -1.0;
  for (const Cand& c : cands) {
    const int64_t tiles = ((M + c.t.bm - 1) / c.t.bm) * ((N + c.t.bn - 1) / c.t.bn);
    const int64_t slots = 256 * (int64_t)c.per_cu;
    const double rounds = (double)tiles / (double)slots;
    const double fill = rounds / (double)((tiles + slots - 1) / slots);
    const double score = fill * c.eff;
    if (score > best_score + 1e-9) {
      best_score = score;
      best = c.t;
    }
  }
  return best;
}

template <int BM, int BN, int WM, int WN, int ODT>
hipError_t launch_dma(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                      int64_t M, int64_t N, int64_t K, void* out, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL((w4a4_gemm_dma_kernel<BM, BN, WM, WN, 3, (BM * BN < 65536), ODT>), dim3((unsigned)(tm * tn)), dim3(WM * WN * 64),
                     0, stream, (const int8_t*)act, xs, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks,
                     tm, tn);
  return hipGetLastError();
}

template <bool APACK, int ODT>
hipError_t launch_t(const void* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                    int64_t M, int64_t N, int64_t K, void* out, hipStream_t stream) {
  const Tile t = choose_tile(M, N);
  if constexpr (!APACK) {
    if (!getenv("CONVROT_GEMM_NO_DMA")) {
#define CONVROT_DMA(BM_, BN_, WM_, WN_)                        \
  if (t.bm == BM_ && t.bn == BN_ && t.wm == WM_ && t.wn == WN_) \
    return launch_dma<BM_, BN_, WM_, WN_, ODT>(act, xs, wq, ws, bias, M, N, K, out, stream);
      CONVROT_DMA(256, 256, 2, 4)
      CONVROT_DMA(256, 128, 4, 2)
      CONVROT_DMA(128, 256, 2, 4)
      CONVROT_DMA(128, 128, 2, 2)
#undef CONVROT_DMA
    }
  }
#define CONVROT_TILE(BM_, BN_, WM_, WN_)                    \
  if (t.bm == BM_ && t.bn == BN_ && t.wm == WM_ && t.wn == WN_) \
    return launch_tile<BM_, BN_, WM_, WN_, APACK, ODT>(act, xs, wq, ws, bias, M, N, K, out, stream);
  CONVROT_TILE(256, 256, 2, 4)
  CONVROT_TILE(256, 256, 4, 2)
  CONVROT_TILE(256, 256, 2, 2)
  CONVROT_TILE(256, 128, 2, 2)
  CONVROT_TILE(256, 128, 4, 2)
  CONVROT_TILE(128, 256, 2, 2)
  CONVROT_TILE(128, 256, 2, 4)
#undef CONVROT_TILE
  return launch_tile<128, 128, 2, 2, APACK, ODT>(act, xs, wq, ws, bias, M, N, K, out, stream);
}

template <bool APACK>
hipError_t launch_odt(int odt, const void* act, const float* xs, const uint8_t* wq, const float* ws,
                      const float* bias, int64_t M, int64_t N, int64_t K, void* out, hipStream_t stream) {
  switch (odt) {
    case kF32: return launch_t<APACK, kF32>(act, xs, wq, ws, bias, M, N, K, out, stream);
    case kF16: return launch_t<APACK, kF16>(act, xs, wq, ws, bias, M, N, K, out, stream);
    default: return launch_t<APACK, kBF16>(act, xs, wq, ws, bias, M, N, K, out, stream);
  }
}

}  // namespace

hipError_t launch_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                            const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  if (act_format == CONVROT_ACT_PACKED)
    return launch_odt<true>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, stream);
  return launch_odt<false>(out_dtype, act, xscales, qweight, wscales, bias, M, N, K, out, stream);
}

}  // namespace convrot
