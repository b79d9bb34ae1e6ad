// W4A4 GEMM for few token rows on gfx950: int8 A4 activation codes x packed
// signed int4 weights on 16x16x64 i8 MFMA, exact int32 accumulation, and the
// same fused epilogue as the tiled kernel, ((f(dot) * xs) * ws) + bias.
//
// Serves mpp_w4a4_int8_matmul (/root/reference/src/convrot_mlx/core.py:1088-1120)
// when M is small -- in a diffusion transformer the adaLN modulation rows
// (M = batch) -- where the tiled kernel's 128-row tiles leave the MFMAs idle
// and one tile column per CU cannot stream the weights fast enough.  Like the
// W4A16 kernel, every weight byte is read from HBM once (16-byte loads of 1 KB
// CDNA4 blocks) and each wave issues all loads of its KPW k-blocks before its
// first MFMA.  Nibbles expand to 16x-scaled int8 codes (two VALU ops per 8
// codes), the MFMA sums are 16x the integer dot exactly, and the dot is
// recovered by an exact shift; integer partial sums of the SPLIT waves are
// added through LDS.  The result is bit-identical to the tiled kernel's.
//
// Ragged edges need no masking: weight blocks past K are zero-padded in the
// CDNA4 layout, so whatever int8 values the activation loads return there
// contribute exactly 0; activation rows past M and reads past either buffer
// return zeros through the buffer range check; output rows >= M and columns
// >= N are not stored.
#include <stdlib.h>

#include "convrot_device.h"
#include "convrot_launch.h"

namespace convrot {
namespace {

// Work split: a workgroup owns NB consecutive 16-column weight tiles and 16*FM
// token rows; wave w takes k-blocks w*KPW .. w*KPW+KPW-1, then every SPLIT*KPW.
template <int ODT, int FM, int NB, int SPLIT, int KPW>
__global__ __launch_bounds__(SPLIT * 64) __attribute__((amdgpu_waves_per_eu(FM == 1 ? 4 : 1)))
void w4a4_smallm_kernel(const int8_t* __restrict__ act, const float* __restrict__ xscales,
                        const uint8_t* __restrict__ wq, const float* __restrict__ wscales,
                        const float* __restrict__ bias, void* __restrict__ out, int M, int N, int K, int nblocks,
                        int kblocks, GatedResidual gr) {
  __shared__ __attribute__((aligned(16))) i32x4 red[SPLIT > 1 ? SPLIT : 1][NB * FM][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb0 = blockIdx.x * NB;
  const int m0 = blockIdx.y * 16 * FM;
  const int q = lane >> 4, r = lane & 15;

  i32x4 acc[NB][FM];
#pragma unroll
  for (int a = 0; a < NB; ++a)
#pragma unroll
    for (int b = 0; b < FM; ++b) acc[a][b] = (i32x4){0, 0, 0, 0};

  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int rows_valid = min(16 * FM, M - m0);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(act + (int64_t)m0 * K), (short)0, rows_valid * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(wq + (int64_t)nb0 * 1024), (short)0, (int)(((int64_t)kblocks * nblocks - nb0) * 1024), 0x00020000);
  for (int kb0 = wave * KPW; kb0 < kblocks; kb0 += SPLIT * KPW) {
    uint4 w[KPW][NB];
    i32x4 aop[KPW][FM][2];  // lane (row r, q): features kb*128 + 32q + 16ks .. +16
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const uint32_t kb = (uint32_t)(kb0 + i);
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
            rw, (int)((kb * (uint32_t)nblocks + (uint32_t)t) * 1024u + (uint32_t)lane * 16u), 0, 0);
        w[i][t] = make_uint4(v.x, v.y, v.z, v.w);
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
              ra, (int)((uint32_t)(fm * 16 + r) * (uint32_t)K + kb * 128u + (uint32_t)(32 * q + 16 * ks)), 0, 0);
          aop[i][fm][ks] = (i32x4){(int)v.x, (int)v.y, (int)v.z, (int)v.w};
        }
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i)
#pragma unroll
      for (int t = 0; t < NB; ++t)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          uint32_t l0, h0, l1, h1;
          nibbles_x16(ks ? w[i][t].z : w[i][t].x, l0, h0);
          nibbles_x16(ks ? w[i][t].w : w[i][t].y, l1, h1);
          const i32x4 bop = (i32x4){(int)l0, (int)h0, (int)l1, (int)h1};
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
            acc[t][fm] = __builtin_amdgcn_mfma_i32_16x16x64_i8(bop, aop[i][fm][ks], acc[t][fm], 0, 0, 0);
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
        i32x4 s = red[0][t * FM + fm][lane];
        for (int w2 = 1; w2 < SPLIT; ++w2) s += red[w2][t * FM + fm][lane];
        acc[t][fm] = s;
      }
  }

  // ---- epilogue (core.py:1168-1170 order): ((f(dot) * xs) * ws) + bias, one rounding per op,
  // then the optional gated residual
  const bool vec_ok = (N & 3) == 0;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = m0 + fm * 16 + r;
    if (m >= M) continue;
    const float xs = xscales[m];
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int n = (nb0 + t) * 16 + 4 * q;
      if (n >= N) continue;
      float o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int nn = n + j < N ? n + j : N - 1;
        o[j] = (((float)(acc[t][fm][j] >> 4) * xs) * wscales[nn]) + (bias ? bias[nn] : 0.0f);
      }
      // One fragment at a time: holding the operands of all FM x NB fragments
      // raises the register count (and lowers occupancy) of every launch.
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

template <int ODT, int FM, int NB, int SPLIT, int KPW>
hipError_t launch_t(const int8_t* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                    int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  dim3 grid((unsigned)((nblocks + NB - 1) / NB), (unsigned)((M + 16 * FM - 1) / (16 * FM)));
  hipLaunchKernelGGL((w4a4_smallm_kernel<ODT, FM, NB, SPLIT, KPW>), grid, dim3(64 * SPLIT), 0, stream, act, xs, wq,
                     ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks, gr);
  return hipGetLastError();
}

// Configurations (FM token tiles, NB weight tiles, SPLIT waves, KPW blocks per
// wave), measured on MI355X over M = 1 .. 64 and the FLUX modulation / MLP
// shapes (K = 3072 -> N = 3072 .. 18432, and 12288 -> 3072), timed from HIP
// graph replays with the weights cycled through > 512 MB:
//   A (1,2,8,3)   M <= 32, many weight tiles (N > 4096)
//   B (1,1,16,4)  M <= 16, few weight tiles (long K per tile)
//   C (2,2,8,2)   32 < M <= 64
//   F (4,2,4,2)   sweeps and tests only
// At M = 1, 3072 -> 18432 (28.3 MB of int4 weights) takes 9.9 us (2.9 TB/s)
// against 17.4 us in the tiled kernel.  The w4a4_smallm_cfg tuning override
// (A|B|C|F) forces the choice.
template <int ODT>
hipError_t launch_shape(const int8_t* act, const float* xs, const uint8_t* wq, const float* ws, const float* bias,
                        int64_t M, int64_t N, int64_t K, void* out, const GatedResidual& gr, hipStream_t stream) {
  const int64_t nblocks = (N + 15) / 16;
  char cfg = M > 32 ? 'C' : (M <= 16 && nblocks <= 256 ? 'B' : 'A');
  if (const int v = tuning(kTuneW4a4SmallmCfg); v == 'A' || v == 'B' || v == 'C' || v == 'F') cfg = (char)v;
  switch (cfg) {
    case 'A': return launch_t<ODT, 1, 2, 8, 3>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    case 'B': return launch_t<ODT, 1, 1, 16, 4>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    case 'C': return launch_t<ODT, 2, 2, 8, 2>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
    default: return launch_t<ODT, 4, 2, 4, 2>(act, xs, wq, ws, bias, M, N, K, out, gr, stream);
  }
}

}  // namespace

hipError_t launch_w4a4_smallm(const int8_t* act, const float* xscales, const uint8_t* qweight,
                              const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K, void* out,
                              int out_dtype, hipStream_t stream, const GatedResidual& gr) {
  if (M == 0 || N == 0) return hipSuccess;
  switch (out_dtype) {
    case kF32: return launch_shape<kF32>(act, xscales, qweight, wscales, bias, M, N, K, out, gr, stream);
    case kF16: return launch_shape<kF16>(act, xscales, qweight, wscales, bias, M, N, K, out, gr, stream);
    default: return launch_shape<kBF16>(act, xscales, qweight, wscales, bias, M, N, K, out, gr, stream);
  }
}

}  // namespace convrot
