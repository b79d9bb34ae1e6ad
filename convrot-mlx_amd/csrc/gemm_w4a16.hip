// W4A16 GEMM for gfx950: rotated bf16/f16 activations x packed signed int4
// weights on 16x16x32 bf16/f16 MFMA, float32 accumulation, fused epilogue.
//
// Replaces the reference's MPP float x int4 TensorOp (/root/reference/src/
// convrot_mlx/core.py:877-912, launched by mpp_w4a16_matmul :1123-1150) and its
// elementwise epilogue `(dots * wscales + bias).astype(dtype)` (:1151-1152).
// Built for the small-M, weight-bandwidth-bound regime: every weight byte is
// read from HBM once (16-byte loads of 1 KB CDNA4 blocks); each wave expands
// its nibbles to 16x-scaled bf16/f16 codes in registers (exact: |16k| <= 128)
// and the 1/16 is folded into the weight scale, so the float32 products and
// sums are exactly 16x those of unscaled codes.
//
// Work split: a workgroup owns NB consecutive 16-row weight tiles and a tile
// of 16*FM tokens; its SPLIT waves take KPW consecutive 128-feature blocks of
// K each (then every SPLIT*KPW) and their partial sums are reduced through
// LDS in a fixed order (deterministic).  A wave issues every load of its KPW
// blocks before the first MFMA: at these M the kernel streams the weights
// from HBM, and the whole matrix has to be in flight at once to cover the
// memory latency (18.9 MB for 3072x12288).
#include <stdlib.h>

#include "convrot_device.h"
#include "convrot_launch.h"

namespace convrot {
namespace {

// 8 codes of one CDNA4 weight dword (byte j: feature j low nibble, j+4 high
// nibble) as 16x-scaled 16-bit floats, natural feature order.
template <int ADT>
__device__ __forceinline__ i32x4 expand8(uint32_t w) {
  uint32_t lo, hi;
  nibbles_x16(w, lo, hi);
  float f[8];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    f[j] = (float)(int8_t)(lo >> (8 * j));
    f[4 + j] = (float)(int8_t)(hi >> (8 * j));
  }
  i32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[j] = (int)(ADT == kBF16 ? pack_bf16x2(f[2 * j], f[2 * j + 1]) : pack_f16x2(f[2 * j], f[2 * j + 1]));
  }
  return r;
}

// Activation fragments of one 128-feature block.  Load c gives lane
// L = 16 u1 + 4 u0 + j the 8 features 32 u1 + 8 j .. +7 of token row
// 4 u0 + c, so the 16 lanes of each 4-lane quad group read a row's 256
// contiguous bytes (the MFMA layout, lane 16q + r holding row r, would put a
// row's 64 bytes in lanes 16 apart, one cache access per lane).  The MFMA
// wants lane 16q + r to hold features 32q + 8s .. +7 of row r in a[s]: with
// q = u1 and r = 4 u0 + c that is the 4 x 4 transpose of (lane bits 0-1,
// slot) inside every quad.  It goes through the wave's own 4160-byte LDS
// buffer: load c's registers at byte c * 1040 + 16 L (contiguous writes), and
// lane 16q + r reads slot s from (r & 3) * 1040 + 16 (16q + 4 (r >> 2) + s).
// The 1040-byte stride puts the 16 rows a read instruction's 16-lane group
// touches in 16 different 16-byte bank groups.
constexpr int kXposeStride = 1040, kXposeBytes = 4 * kXposeStride;

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void transpose_quads4(i32x4 (&a)[4], uint8_t* buf, int lane) {
  const int q = lane >> 4, r = lane & 15;
#pragma unroll
  for (int c = 0; c < 4; ++c) *(i32x4*)(buf + c * kXposeStride + lane * 16) = a[c];
  wave_lds_fence();
#pragma unroll
  for (int s = 0; s < 4; ++s) a[s] = *(const i32x4*)(buf + (r & 3) * kXposeStride + (16 * q + 4 * (r >> 2) + s) * 16);
  wave_lds_fence();  // the buffer's next writes come after these reads
}

template <int ADT>
__device__ __forceinline__ f32x4 mfma16(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (ADT == kBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Split of K over workgroups (grid.z): workgroup z takes the k-blocks
// [z * kspan, (z + 1) * kspan).  part: float32 partial fragments, NB * FM of
// 1 KB (16 bytes a lane) per (group, split), group = blockIdx.y * gridDim.x +
// blockIdx.x; ctr: the group's arrival counter at ctr[32 * group] (zero
// before the launch, zero again after it).  gridDim.x is a multiple of the 8
// XCDs, so the splits of a group (linear workgroup ids x + gridDim.x * z,
// dispatched round-robin to the XCDs) all run on one XCD and share its L2;
// the groups past the weight tiles exit at once.
struct SplitK {
  uint8_t* part = nullptr;
  int* ctr = nullptr;
  int splits = 1;
  int kspan = 0;
};

// Single token tile: four waves per SIMD (at most 128 VGPRs), so that the
// whole grid's weight loads can be in flight at once.
template <int ADT, int ODT, int FM, int NB, int SPLIT, int KPW, bool QL, bool SK = false>
__global__ __launch_bounds__(SPLIT * 64) __attribute__((amdgpu_waves_per_eu(FM == 1 ? 4 : 1)))
void w4a16_gemm_kernel(const uint16_t* __restrict__ act, const uint8_t* __restrict__ wq,
                       const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out,
                       int M, int N, int K, int nblocks, int kblocks, GatedResidual gr, SplitK sk) {
  __shared__ __attribute__((aligned(16))) f32x4 red[SPLIT > 1 ? SPLIT : 1][NB * FM][64];
  __shared__ __attribute__((aligned(16))) uint8_t xpose[QL ? SPLIT * kXposeBytes : 16];  // per-wave buffers
  __shared__ float epi[2][NB * 16];  // the epilogue's weight scales and bias
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb0 = blockIdx.x * NB;
  const int m0 = blockIdx.y * 16 * FM;
  const int q = lane >> 4, r = lane & 15;
  if (SK && nb0 >= nblocks) return;  // XCD padding (whole workgroup)

  // Wave 0, which alone runs the epilogue, loads the tile's weight scales and
  // bias before the weights, so that their round trip does not follow the
  // reduction (0.5-0.8 us of a ~8 us launch at 3072 -> 12288).  Columns past
  // N read column N - 1, as the epilogue's clamped index does.
  float pre_ws = 0.0f, pre_b = 0.0f;
  if (wave == 0 && lane < NB * 16) {
    const int nn = min(nb0 * 16 + lane, N - 1);
    pre_ws = wscales[nn];
    pre_b = bias ? bias[nn] : 0.0f;
  }

  f32x4 acc[NB][FM];
#pragma unroll
  for (int a = 0; a < NB; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // Branch-free loads through buffer resources (the range check zero-fills
  // past the end), so the compiler can wait for each block separately and the
  // weight expansion of early blocks overlaps the later loads.  Weight tile
  // rows past N read wrapped (valid) blocks; their outputs are never stored.
  // Activation rows are based at m0 (32-bit offsets for any M).
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int rows_valid = min(16 * FM, M - m0);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(act + (int64_t)m0 * K), (short)0, rows_valid * K * 2, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(wq + (int64_t)nb0 * 1024), (short)0, (int)(((int64_t)kblocks * nblocks - nb0) * 1024), 0x00020000);
  const int kb_lo = SK ? (int)blockIdx.z * sk.kspan : 0;
  const int kb_hi = SK ? min(kb_lo + sk.kspan, kblocks) : kblocks;
  for (int kb0 = kb_lo + wave * KPW; kb0 < kb_hi; kb0 += SPLIT * KPW) {
    uint4 w[KPW][NB];
    i32x4 aop[KPW][FM][4];  // lane (q, r) -> 8 values at features kb*128 + 32q + 8c of row r (after QL's transpose)
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      // blocks at or past kblocks read zeros; with SK so do the blocks at or
      // past kb_hi, which belong to the next split (offset past the range)
      const int kb = kb0 + i;
      const bool kin = !SK || kb < kb_hi;
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const uint32_t off = ((uint32_t)kb * (uint32_t)nblocks + (uint32_t)t) * 1024u + (uint32_t)lane * 16u;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(rw, (int)(kin ? off : 0x80000000u), 0, 0);
        w[i][t] = make_uint4(v.x, v.y, v.z, v.w);
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          // QL: quad-coalesced order (transposed before use); else the MFMA
          // order, lane (q, r) reading row r, features 32q + 8c (a token
          // row's 64 bytes spread over lanes 16 apart)
          const int k = QL ? kb * 128 + 32 * q + 8 * (lane & 3) : kb * 128 + 32 * q + 8 * c;
          const int row = QL ? fm * 16 + 4 * ((lane >> 2) & 3) + c : fm * 16 + r;
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
              ra, (int)((uint32_t)row * (uint32_t)K * 2u + (uint32_t)k * 2u), 0, 0);
          // a ragged K end would read the next row: zero it (K is a multiple of 8)
          aop[i][fm][c] = k < K && kin ? (i32x4){(int)v.x, (int)v.y, (int)v.z, (int)v.w} : (i32x4){0, 0, 0, 0};
        }
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        if constexpr (QL) transpose_quads4(aop[i][fm], xpose + wave * kXposeBytes, lane);
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const uint32_t wd[4] = {w[i][t].x, w[i][t].y, w[i][t].z, w[i][t].w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const i32x4 bop = expand8<ADT>(wd[c]);
#pragma unroll
          for (int fm = 0; fm < FM; ++fm) acc[t][fm] = mfma16<ADT>(bop, aop[i][fm][c], acc[t][fm]);
        }
      }
    }
  }

  if constexpr (SPLIT > 1) {
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) red[wave][t * FM + fm][lane] = acc[t][fm];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        f32x4 s = red[0][t * FM + fm][lane];
        for (int w2 = 1; w2 < SPLIT; ++w2) s += red[w2][t * FM + fm][lane];
        acc[t][fm] = s;
      }
  }

  if constexpr (SK) {
    // Store this split's partial (device-scope stores), then count the
    // arrival once they are complete; the group's last arrival adds all its
    // partials in split order (the same sum whichever split arrives last),
    // rearms the counter and runs the epilogue.  No workgroup waits for another.
    const int grp = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    constexpr int NF = NB * FM;
    uint8_t* const gbase = sk.part + (size_t)grp * sk.splits * (NF * 1024) + lane * 16;
    uint64_t* const mine = (uint64_t*)(gbase + (size_t)blockIdx.z * (NF * 1024));
#pragma unroll
    for (int t = 0; t < NB; ++t)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const f32x4 a = acc[t][fm];
        uint64_t* const p = mine + (t * FM + fm) * 128;
        __hip_atomic_store(p, (uint64_t)__float_as_uint(a[0]) | ((uint64_t)__float_as_uint(a[1]) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(p + 1, (uint64_t)__float_as_uint(a[2]) | ((uint64_t)__float_as_uint(a[3]) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    wait_vmcnt<0>();
    int arrived = 0;
    if (lane == 0) arrived = atomicAdd(&sk.ctr[32 * grp], 1);
    if (__builtin_amdgcn_readlane(arrived, 0) != sk.splits - 1) return;
    if (lane == 0) __hip_atomic_store(&sk.ctr[32 * grp], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int z = 0; z < sk.splits; ++z) {
      i32x4 v[NF];
#pragma unroll
      for (int f = 0; f < NF; ++f) v[f] = load_dev16<0>(gbase + ((size_t)z * NF + f) * 1024);
      wait_vmcnt<0>();
#pragma unroll
      for (int f = 0; f < NF; ++f) {
        asm volatile("" : "+v"(v[f]));  // the adds stay behind the wait
        const f32x4 p = __builtin_bit_cast(f32x4, v[f]);
        acc[f / FM][f % FM] = z == 0 ? p : acc[f / FM][f % FM] + p;
      }
    }
  }

  // ---- epilogue (core.py:1151-1152): (dots * ws) + bias, rounded once
  if (lane < NB * 16) {  // wave 0 writes and reads these: LDS keeps its order
    epi[0][lane] = pre_ws;
    epi[1][lane] = pre_b;
  }
  const bool vec_ok = (N & 3) == 0;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = m0 + fm * 16 + r;
    if (m >= M) continue;
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int n = (nb0 + t) * 16 + 4 * q;
      if (n >= N) continue;
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = t * 16 + 4 * q + j;  // column n + j (clamped to N - 1 at load)
        float v = acc[t][fm][j] * (epi[0][c] * 0.0625f);  // codes were scaled by 16
        v = v + epi[1][c];
        o[j] = v;
      }
      if (gr.residual) gate_residual4<ODT>(gr, m, n, N, vec_ok, o);
      const int64_t idx = (int64_t)m * N + n;
      if (vec_ok) {
        store_out4<ODT>(out, idx, o[0], o[1], o[2], o[3]);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (n + j < N) store_out<ODT>(out, idx + j, o[j]);
      }
    }
  }
}

// ---- many token rows: tiled kernel on direct-to-LDS loads
//
// A workgroup of 8 waves owns a BM (tokens) x BN (output features) tile,
// BM, BN in {128, 256}; wave w computes rows (w / 4) * BM/2 .. and features
// (w % 4) * BN/4 .. as FM x FN float32 fragments of 16 x 16.  K advances in
// 128-feature blocks through two LDS stages, each filled by one-KB
// buffer_load ... lds pieces (no register staging):
//   activations: BM rows x 256 bytes; piece j = rows 4j .. 4j+3, lane L
//     writes row 4j + L/16, slot L%16, which receives the row's 16-byte chunk
//     (L%16) ^ (row & 15): 16 lanes reading one chunk of 16 consecutive rows
//     then hit 16 different bank groups;
//   weights: BN/16 CDNA4 blocks (16 features x 128 k each) read as stored.
// Block i+1 is loaded while block i is multiplied.  Per k-step of 32 the
// wave expands its FN weight fragments (8 codes per lane) to 16x-scaled
// 16-bit floats once and uses each for FM MFMAs.  Rows >= M and reads past
// the weights return zeros (buffer range check); the ragged end of K is
// zeroed at the fragment (K % 8 == 0, so fragments are whole or empty).
constexpr int kTileWaves = 8;

template <int BM, int BN>
struct TiledShape {
  static constexpr int FM = BM / 32, FN = BN / 64;           // 16x16 fragments per wave
  static constexpr int APieces = BM / 4, BPieces = BN / 16;  // one-KB pieces per stage
  static constexpr int APW = APieces / kTileWaves, BPW = BPieces / kTileWaves;
  static constexpr int StageBytes = (APieces + BPieces) * 1024;
  static constexpr int RS = BN / 2 + 16;  // output staging row: BN/4 16-bit values + 16 bytes
  static_assert(APW * kTileWaves == APieces && BPW * kTileWaves == BPieces, "pieces split over waves");
  static_assert(kTileWaves * (BM / 2) * RS <= 2 * StageBytes, "output staging fits the ring");
};

template <int ADT, int ODT, int BM, int BN>
__global__ __launch_bounds__(kTileWaves * 64) __attribute__((amdgpu_waves_per_eu(BM * BN <= 128 * 128 ? 4 : 2)))
void w4a16_tiled_kernel(const uint16_t* __restrict__ act, const uint8_t* __restrict__ wq,
                        const float* __restrict__ wscales, const float* __restrict__ bias, void* __restrict__ out,
                        int M, int N, int K, int nblocks, int kblocks, int tiles_m, int tiles_n, GatedResidual gr) {
  using S = TiledShape<BM, BN>;
  constexpr int FM = S::FM, FN = S::FN;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * S::StageBytes];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / 4, wn = wave % 4;
  const int q = lane >> 4, r = lane & 15;

  // Tile order: consecutive workgroups of one XCD take adjacent tiles, four
  // tile rows at a time (they share activation rows and weight columns in L2).
  const int tiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  const int per_xcd = tiles / 8;
  if (t < per_xcd * 8) t = (t % 8) * per_xcd + t / 8;
  const int gm = t / (4 * tiles_n), first = gm * 4, rows_g = min(4, tiles_m - first);
  const int in_g = t - gm * 4 * tiles_n;
  const int m0 = (first + in_g % rows_g) * BM, n0 = (in_g / rows_g) * BN;

  const int rows_valid = min(BM, M - m0);
  const i32x4_sgpr ra = buffer_rsrc(act + (int64_t)m0 * K, (uint32_t)rows_valid * (uint32_t)K * 2u);
  const i32x4_sgpr rw = buffer_rsrc(wq + (int64_t)(n0 / 16) * 1024,
                                    (uint32_t)(((int64_t)kblocks * nblocks - n0 / 16) * 1024));
  const uint32_t smem_addr = (uint32_t)(uintptr_t)smem;
  // this lane's activation piece offsets: row 4j + L/16 of a piece, and
  // (4j + L/16) & 15 = 4 (j & 3) + L/16
  uint32_t va[4];
#pragma unroll
  for (int j4 = 0; j4 < 4; ++j4) {
    const int row = 4 * j4 + (lane >> 4);
    va[j4] = (uint32_t)(row * K * 2 + 16 * ((lane & 15) ^ row));
  }
  auto issue = [&](int kb, int stage) {
    const uint32_t base = smem_addr + (uint32_t)(stage * S::StageBytes);
#pragma unroll
    for (int i = 0; i < S::APW; ++i) {
      const uint32_t j = (uint32_t)(wave * S::APW + i);
      uint32_t so = (j & ~3u) * 4u * (uint32_t)K * 2u + (uint32_t)kb * 256u;  // rows 4j.., block kb
      asm volatile("" : "+s"(so));
      dma16(ra, va[j & 3] + so, base + j * 1024u);
    }
#pragma unroll
    for (int i = 0; i < S::BPW; ++i) {
      const uint32_t j = (uint32_t)(wave * S::BPW + i);
      uint32_t so = j * 1024u + (uint32_t)kb * (uint32_t)nblocks * 1024u;
      asm volatile("" : "+s"(so));
      dma16(rw, (uint32_t)lane * 16u + so, base + (uint32_t)(S::APieces + j) * 1024u);
    }
  };

  f32x4 acc[FN][FM];
#pragma unroll
  for (int a = 0; a < FN; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (f32x4){0.f, 0.f, 0.f, 0.f};

  const bool ragged = (K & 127) != 0;
  issue(0, 0);
  for (int i = 0; i < kblocks; ++i) {
    wait_vmcnt<0>();
    __syncthreads();  // block i visible; every wave is done with stage (i + 1) % 2
    if (i + 1 < kblocks) issue(i + 1, (i + 1) & 1);
    const uint8_t* st = smem + (i & 1) * S::StageBytes;
    uint4 wd[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
      wd[fn] = *(const uint4*)(st + (S::APieces + wn * FN + fn) * 1024 + lane * 16);
    const bool last = ragged && i + 1 == kblocks;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      i32x4 aop[FM];
      const int chunk = 4 * q + c;  // features 32q + 8c .. +7 of the block
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * (BM / 2) + fm * 16 + r;
        aop[fm] = *(const i32x4*)(st + row * 256 + 16 * (chunk ^ r));
      }
      if (last && i * 128 + 8 * chunk >= K) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) aop[fm] = (i32x4){0, 0, 0, 0};
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const uint32_t wdc = c == 0 ? wd[fn].x : c == 1 ? wd[fn].y : c == 2 ? wd[fn].z : wd[fn].w;
        const i32x4 bop = expand8<ADT>(wdc);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) acc[fn][fm] = mfma16<ADT>(bop, aop[fm], acc[fn][fm]);
      }
    }
  }
  __syncthreads();  // ring -> output staging

  // ---- epilogue (core.py:1151-1152): (dots * ws) + bias, rounded once; codes were scaled by 16
  const int mw = m0 + wm * (BM / 2), nw = n0 + wn * (BN / 4);
  if constexpr (ODT == kF32) {
    const bool vec_ok = (N & 3) == 0;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int n = nw + fn * 16 + 4 * q;
      if (n >= N) continue;
      float wsv[4], bv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nn = n + j < N ? n + j : N - 1;
        wsv[j] = wscales[nn] * 0.0625f;
        bv[j] = bias ? bias[nn] : 0.0f;
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int m = mw + fm * 16 + r;
        if (m >= M) continue;
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = acc[fn][fm][j] * wsv[j] + bv[j];
        if (gr.residual) gate_residual4<ODT>(gr, m, n, N, vec_ok, o);
        const int64_t idx = (int64_t)m * N + n;
        if (vec_ok) {
          store_out4<ODT>(out, idx, o[0], o[1], o[2], o[3]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (n + j < N) store_out<ODT>(out, idx + j, o[j]);
        }
      }
    }
  } else {
    // 16-bit outputs go through the wave's LDS region (BM/2 rows of RS bytes)
    // and leave as 16-byte stores of whole row segments.
    uint8_t* region = smem + wave * (BM / 2) * S::RS;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int nl = fn * 16 + 4 * q;
      float wsv[4], bv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nn = min(nw + nl + j, N - 1);
        wsv[j] = wscales[nn] * 0.0625f;
        bv[j] = bias ? bias[nn] : 0.0f;
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        float o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = acc[fn][fm][j] * wsv[j] + bv[j];
        const uint2 w2 = ODT == kBF16 ? make_uint2(pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]))
                                      : make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
        *(uint2*)(region + (fm * 16 + r) * S::RS + nl * 2) = w2;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int CPR = BN / 32;         // 16-byte chunks per staged row
    constexpr int RPI = 64 / CPR;        // rows per instruction
    constexpr int NIT = (BM / 2) / RPI;  // write-back iterations
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
        store_row(it, *(const uint4*)(region + rl * S::RS + cc * 16));
      }
    } else {
      // Gated residual: the residual / gate loads of BATCH rows go out before
      // their stores (a load cannot move above a store that may alias it).
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
          store_row(b0 + i, gate_apply8<ODT>(ops[i], *(const uint4*)(region + rl * S::RS + cc * 16)));
        }
      }
    }
  }
}

template <int ADT, int ODT, int BM, int BN>
hipError_t launch_tiled_t(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                          int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int tm = (int)((M + BM - 1) / BM), tn = (int)((N + BN - 1) / BN);
  hipLaunchKernelGGL((w4a16_tiled_kernel<ADT, ODT, BM, BN>), dim3((unsigned)(tm * tn)), dim3(kTileWaves * 64), 0,
                     stream, (const uint16_t*)act, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, tm,
                     tn, gr);
  return hipGetLastError();
}

// Tile choice: the candidate with the least modelled time.  Each CU works
// through ceil(tiles / CUs) tiles of BM * BN * kblocks MFMA work at the tile's
// rate, holding per_cu of them at once, plus a fixed cost (pipeline fill and
// epilogue) per resident batch.  Rates and the fixed cost (in units of one
// 128-feature block of a 256 x 256 tile, ~4 us) are fitted to MI355X timings
// of M = 512 .. 4096, K = 3072 .. 15360, N = 3072 .. 21504: a 128 x 128 tile
// (two per CU) sustains the 256 x 256 tile's throughput and wins whenever the
// 256 x 256 grid leaves CUs idle or has a partial last round.
// The w4a16_tile tuning override (256x256, 256x128, 128x256 or 128x128) forces one.
struct TiledCand {
  int bm, bn, per_cu;
  double rate;
};
constexpr TiledCand kTiledCands[] = {
    {256, 256, 1, 1.00},
    {256, 128, 1, 0.85},
    {128, 256, 1, 0.75},
    {128, 128, 2, 1.00},
};
constexpr double kTiledFixed = 1.5;
constexpr double kTiledUsPerUnit = 4.0;

struct TiledPlan {
  int pick;   // index into kTiledCands
  double us;  // modelled launch time
};

TiledPlan tiled_plan(int64_t M, int64_t N, int64_t K) {
  const int64_t cus = device_cus();
  const int64_t kb = (K + 127) / 128;
  int bm = 0, bn = 0;
  if (const int v = tuning(kTuneW4a16Tile); v >= 0) bm = v & 1023, bn = (v >> 10) & 1023;
  TiledPlan best{3, 1e300};
  for (int i = 0; i < (int)(sizeof(kTiledCands) / sizeof(kTiledCands[0])); ++i) {
    const TiledCand& c = kTiledCands[i];
    if (bm && (c.bm != bm || c.bn != bn)) continue;
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn);
    const int64_t per_cu = (tiles + cus - 1) / cus;
    const double units = (double)per_cu * ((double)c.bm * c.bn / 65536.0 * (double)kb) / c.rate +
                         kTiledFixed * (double)((per_cu + c.per_cu - 1) / c.per_cu);
    if (units * kTiledUsPerUnit < best.us) best = {i, units * kTiledUsPerUnit};
  }
  return best;
}

template <int ADT, int ODT>
hipError_t launch_tiled(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                        int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int pick = tiled_plan(M, N, K).pick;
  switch (pick) {
    case 0: return launch_tiled_t<ADT, ODT, 256, 256>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 1: return launch_tiled_t<ADT, ODT, 256, 128>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 2: return launch_tiled_t<ADT, ODT, 128, 256>(act, wq, ws, bias, M, N, K, out, gr, stream);
    default: return launch_tiled_t<ADT, ODT, 128, 128>(act, wq, ws, bias, M, N, K, out, gr, stream);
  }
}

template <int ADT, int ODT, int FM, int NB, int SPLIT, int KPW, bool QL>
hipError_t launch_t(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M, int64_t N,
                    int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  dim3 grid((unsigned)((nblocks + NB - 1) / NB), (unsigned)((M + 16 * FM - 1) / (16 * FM)));
  hipLaunchKernelGGL((w4a16_gemm_kernel<ADT, ODT, FM, NB, SPLIT, KPW, QL>), grid, dim3(64 * SPLIT), 0, stream,
                     (const uint16_t*)act, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, gr, SplitK{});
  return hipGetLastError();
}

template <int ADT, int ODT, int FM, int NB, int SPLIT, int KPW, bool QL>
hipError_t launch_sk_t(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M, int64_t N,
                       int64_t K, void* out, const GatedResidual& gr, const SplitK& sk, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  const int groups8 = ((nblocks + NB - 1) / NB + 7) / 8 * 8;
  dim3 grid((unsigned)groups8, (unsigned)((M + 16 * FM - 1) / (16 * FM)), (unsigned)sk.splits);
  hipLaunchKernelGGL((w4a16_gemm_kernel<ADT, ODT, FM, NB, SPLIT, KPW, QL, true>), grid, dim3(64 * SPLIT), 0, stream,
                     (const uint16_t*)act, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, gr, sk);
  return hipGetLastError();
}

// Split-K plan for the weight-streaming kernel: three weight tiles and up to
// 32 token rows (one token tile) per workgroup, eight waves of three k-blocks,
// the k-blocks cut into `splits` ranges so that groups x splits fills the CUs
// once.  Possible at M <= 32 with a workspace, at most kW4a16MaxGroups groups
// of three weight tiles (N <= 4608), at least two splits' worth of groups per
// CU count and K of at least 48 k-blocks: 12288 -> 3072 runs as 64 groups x 4
// splits of 24 k-blocks.  Taken automatically from 9 rows on: the split's
// tail (partial stores acknowledged, the arrival atomic, the partial loads:
// three device-scope round trips) costs more than it saves below that.
// HIP-graph replays, unsplit -> split, 12288 -> 3072: M = 1 8.66 -> 9.82 us,
// M = 8 9.64 -> 10.29, M = 16 11.18 -> 10.62, M = 32 14.25 -> 13.39;
// 15360 -> 3072: M = 8 11.86 -> 11.33, M = 16 13.66 -> 11.84, M = 32
// 16.79 -> 15.01.  `forced` (w4a16_cfg "S") drops the row minimum.
bool w4a16_split_plan(int64_t M, int64_t N, int64_t K, const Workspace& work, bool forced, SplitK* sk) {
  constexpr int kNB = 3, kKS = 8 * 3;
  const int64_t nblocks = (N + 15) / 16, kblocks = (K + 127) / 128;
  const int64_t groups = (nblocks + kNB - 1) / kNB, groups8 = (groups + 7) / 8 * 8;
  if (!work.ptr || M > 32 || (M < 9 && !forced) || kblocks < 2 * kKS || groups8 > kW4a16MaxGroups) return false;
  const int64_t splits_fit = device_cus() / groups;
  if (splits_fit < 2) return false;
  const int64_t kspan = (kblocks + splits_fit - 1) / splits_fit;
  const int64_t splits = (kblocks + kspan - 1) / kspan;
  const int64_t fm = M > 16 ? 2 : 1;
  const size_t part_bytes = (size_t)(groups8 * splits * kNB * fm) * 1024;
  if (kW4a16PartialOffset + part_bytes > work.bytes) return false;
  sk->part = work.ptr + kW4a16PartialOffset;
  sk->ctr = (int*)(work.ptr + kW4a16CounterOffset);
  sk->splits = (int)splits;
  sk->kspan = (int)kspan;
  return true;
}

// Configurations (FM token tiles, NB weight tiles, SPLIT waves, KPW blocks
// per wave), measured on the config-4 shapes (M = 1, 8, 32; 3072->12288 and
// 12288->3072):
//   A (1,2,8,3)  more than 256 weight tiles (N > 4096), or M > 16 unless the
//                tiled kernel is modelled faster
//   B (1,1,16,4) at most 256 weight tiles, M <= 16 (at M = 1: 3072->3072
//                4.3 us vs 4.9, 12288->3072 8.7 vs 12.3; while 3072->6144
//                takes 5.8 us in A against 8.1 in B, whose 16 waves per tile
//                outnumber K = 3072's 24 k-blocks)
//   D (1,3,8,3)  M <= 16 where the weight tiles split into whole rounds of three
//                per workgroup (N = 12288 on 256 CUs)
//   E (2,3,8,2)  17 <= M <= 32 there: both 16-token halves in one workgroup
//   C (2,2,8,2)  sweeps and tests only (one 32-token tile: slower than two of A)
//   F (4,2,4,2)  sweeps and tests only (slower than A at every M measured)
//   T            the tiled kernel (256 / 128 edges), M >= kTiledMinM
//   S            split K over workgroups (1,3,8,3) / (2,3,8,3) where A or B
//                would run and a workspace is given (w4a16_split_plan)
// At M = 1 both stream the 18.9 MB weight matrix in ~8 us (~2.3 TB/s), where
// a plain 19 MB device copy takes ~10 us; the rest is weight expansion
// (~2 VALU ops per code) and the launch/tail.  The w4a16_cfg tuning override
// (A .. F, S, T) forces the kernel (sweeps and tests; S needs a workspace).
constexpr int64_t kTiledMinM = 64;
// From kQuadMinM rows on, splits A and B load activations in the quad-coalesced
// order and transpose them through LDS (transpose_quads4): at M = 16 on the
// config-4 shapes 9.3 against 12.0 us (3072->12288) and 11.2 against 16.8 us
// (12288->3072), at M = 32 12.1 against 15.5 and 15.8 against 19.0.  With a
// few rows the transposes cost more than the scattered loads save: M = 4 runs
// 7.9 against 8.2 us direct (3072->12288) and 8.9 against 9.3 (12288->3072),
// M = 6 8.3 against 8.3 and 9.6 against 9.2.  (The LDS transpose replaced a
// register one of 64 VALU ops per block, which lost up to M = 6; it took M = 32
// from 12.4 to 12.0 us (3072->12288) and 15.8 to 14.4 us (12288->3072),
// bit-identical.)
constexpr int64_t kQuadMinM = 6;
template <int ADT, int ODT>
hipError_t launch_shape(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                        int64_t N, int64_t K, void* out, const GatedResidual& gr, const Workspace& work,
                        hipStream_t stream) {
  const int64_t nblocks = (N + 15) / 16;
  char cfg = (M <= 16 && nblocks <= 256) ? 'B' : 'A';
  // From kTiledMinM rows on, the tiled kernel takes over where its modelled
  // time beats split A's: A runs each 16-token tile at ~246 TFLOP/s over a
  // ~5 us floor, the tiled kernel needs enough tiles to fill the CUs (M = 128:
  // 3072 -> 12288 runs 28 us tiled against 45 us in A; 12288 -> 3072 has 24
  // tiles of long K and stays in A up to M = 256, 78 us against 99 us).
  const double m16 = (double)((M + 15) / 16 * 16);
  if (M >= kTiledMinM && tiled_plan(M, N, K).us < 2.0 * m16 * (double)N * (double)K / 246e6 + 5.0) cfg = 'T';
  // Three weight tiles a workgroup where that makes whole rounds of 256
  // workgroups (N = 12288: 768 tiles), one token tile at up to 16 rows and
  // both 16-row halves of 17 .. 32 rows in one workgroup (every weight byte read
  // once).  Config 4, 3072 -> 12288 (HIP-graph replays, one box): M = 1 7.65
  // against 8.1 us in A, M = 8 8.05 against 8.6, M = 32 10.5 against 12.6.
  if (nblocks % 3 == 0 && (nblocks / 3) % device_cus() == 0 && M <= 32) cfg = M <= 16 ? 'D' : 'E';
  // With a workspace, split K where A or B would leave CUs idle or walk K
  // twice (12288 -> 3072: 192 weight tiles; see w4a16_split_plan).
  const int forced = tuning(kTuneW4a16Cfg);
  SplitK sk;
  if ((forced == 'S' || (forced < 0 && (cfg == 'A' || cfg == 'B'))) &&
      w4a16_split_plan(M, N, K, work, forced == 'S', &sk)) {
    if (M > 16) return launch_sk_t<ADT, ODT, 2, 3, 8, 3, true>(act, wq, ws, bias, M, N, K, out, gr, sk, stream);
    return M >= kQuadMinM ? launch_sk_t<ADT, ODT, 1, 3, 8, 3, true>(act, wq, ws, bias, M, N, K, out, gr, sk, stream)
                          : launch_sk_t<ADT, ODT, 1, 3, 8, 3, false>(act, wq, ws, bias, M, N, K, out, gr, sk, stream);
  }
  if (forced == 'A' || forced == 'B' || forced == 'C' || forced == 'D' || forced == 'E' || forced == 'F' ||
      forced == 'T')
    cfg = (char)forced;
  switch (cfg) {
    case 'T': return launch_tiled<ADT, ODT>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 'D':
      return M >= kQuadMinM ? launch_t<ADT, ODT, 1, 3, 8, 3, true>(act, wq, ws, bias, M, N, K, out, gr, stream)
                            : launch_t<ADT, ODT, 1, 3, 8, 3, false>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 'E': return launch_t<ADT, ODT, 2, 3, 8, 2, true>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 'C': return launch_t<ADT, ODT, 2, 2, 8, 2, true>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 'A':
      return M >= kQuadMinM ? launch_t<ADT, ODT, 1, 2, 8, 3, true>(act, wq, ws, bias, M, N, K, out, gr, stream)
                            : launch_t<ADT, ODT, 1, 2, 8, 3, false>(act, wq, ws, bias, M, N, K, out, gr, stream);
    case 'B':
      return M >= kQuadMinM ? launch_t<ADT, ODT, 1, 1, 16, 4, true>(act, wq, ws, bias, M, N, K, out, gr, stream)
                            : launch_t<ADT, ODT, 1, 1, 16, 4, false>(act, wq, ws, bias, M, N, K, out, gr, stream);
    default: return launch_t<ADT, ODT, 4, 2, 4, 2, true>(act, wq, ws, bias, M, N, K, out, gr, stream);
  }
}

template <int ADT>
hipError_t launch_odt(int odt, const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                      int64_t N, int64_t K, void* out, const GatedResidual& gr, const Workspace& work,
                      hipStream_t stream) {
  switch (odt) {
    case kF32: return launch_shape<ADT, kF32>(act, wq, ws, bias, M, N, K, out, gr, work, stream);
    case kF16: return launch_shape<ADT, kF16>(act, wq, ws, bias, M, N, K, out, gr, work, stream);
    default: return launch_shape<ADT, kBF16>(act, wq, ws, bias, M, N, K, out, gr, work, stream);
  }
}

}  // namespace

hipError_t launch_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                             const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                             hipStream_t stream, const GatedResidual& gr, const Workspace& work) {
  if (M == 0 || N == 0) return hipSuccess;
  if (act_dtype == kF16)
    return launch_odt<kF16>(out_dtype, act, qweight, wscales, bias, M, N, K, out, gr, work, stream);
  return launch_odt<kBF16>(out_dtype, act, qweight, wscales, bias, M, N, K, out, gr, work, stream);
}

bool w4a16_tile_known(int bm, int bn) {
  for (const TiledCand& c : kTiledCands)
    if (c.bm == bm && c.bn == bn) return true;
  return false;
}

}  // namespace convrot
