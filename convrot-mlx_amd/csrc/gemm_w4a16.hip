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

template <int ADT>
__device__ __forceinline__ f32x4 mfma16(i32x4 a, i32x4 b, f32x4 c) {
  if constexpr (ADT == kBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
}

// Single token tile: four waves per SIMD (at most 128 VGPRs), so that the
// whole grid's weight loads can be in flight at once.
template <int ADT, int ODT, int FM, int NB, int SPLIT, int KPW>
__global__ __launch_bounds__(SPLIT * 64) __attribute__((amdgpu_waves_per_eu(FM == 1 ? 4 : 1)))
void w4a16_gemm_kernel(const uint16_t* __restrict__ act,
                                                                const uint8_t* __restrict__ wq,
                                                                const float* __restrict__ wscales,
                                                                const float* __restrict__ bias,
                                                                void* __restrict__ out, int M, int N, int K,
                                                                int nblocks, int kblocks) {
  __shared__ __attribute__((aligned(16))) f32x4 red[SPLIT > 1 ? SPLIT : 1][NB * FM][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb0 = blockIdx.x * NB;
  const int m0 = blockIdx.y * 16 * FM;
  const int q = lane >> 4, r = lane & 15;

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
  for (int kb0 = wave * KPW; kb0 < kblocks; kb0 += SPLIT * KPW) {
    uint4 w[KPW][NB];
    i32x4 aop[KPW][FM][4];  // lane (m = r, q) -> 8 values at features kb*128 + 32q + 8c
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = kb0 + i;  // blocks at or past kblocks read zeros
#pragma unroll
      for (int t = 0; t < NB; ++t) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
            rw, (int)(((uint32_t)kb * (uint32_t)nblocks + (uint32_t)t) * 1024u + (uint32_t)lane * 16u), 0, 0);
        w[i][t] = make_uint4(v.x, v.y, v.z, v.w);
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int k = kb * 128 + 32 * q + 8 * c;
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(
              ra, (int)((uint32_t)(fm * 16 + r) * (uint32_t)K * 2u + (uint32_t)k * 2u), 0, 0);
          // a ragged K end would read the next row: zero it (K is a multiple of 8)
          aop[i][fm][c] = k < K ? (i32x4){(int)v.x, (int)v.y, (int)v.z, (int)v.w} : (i32x4){0, 0, 0, 0};
        }
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i)
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

  // ---- epilogue (core.py:1151-1152): (dots * ws) + bias, rounded once
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
        const int nn = n + j < N ? n + j : N - 1;
        float v = acc[t][fm][j] * (wscales[nn] * 0.0625f);  // codes were scaled by 16
        v = v + (bias ? bias[nn] : 0.0f);
        o[j] = v;
      }
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

template <int ADT, int ODT, int FM, int NB, int SPLIT, int KPW>
hipError_t launch_t(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M, int64_t N,
                    int64_t K, void* out, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  dim3 grid((unsigned)((nblocks + NB - 1) / NB), (unsigned)((M + 16 * FM - 1) / (16 * FM)));
  hipLaunchKernelGGL((w4a16_gemm_kernel<ADT, ODT, FM, NB, SPLIT, KPW>), grid, dim3(64 * SPLIT), 0, stream,
                     (const uint16_t*)act, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks);
  return hipGetLastError();
}

// Configurations (FM token tiles, NB weight tiles, SPLIT waves, KPW blocks
// per wave), measured on the config-4 shapes (M = 1, 8, 32; 3072->12288 and
// 12288->3072):
//   A (1,2,8,3)  many weight tiles, or 16 < M <= 32 (two token tiles)
//   B (1,1,16,4) few weight tiles and long K, M <= 16
//   F (4,2,4,2)  M > 32
// At M = 1 both stream the 18.9 MB weight matrix in ~8 us (~2.3 TB/s), where
// a plain 19 MB device copy takes ~10 us; the rest is weight expansion
// (~2 VALU ops per code) and the launch/tail.  CONVROT_W4A16_CFG=A|B|F
// overrides (tuning sweeps).
template <int ADT, int ODT>
hipError_t launch_shape(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                        int64_t N, int64_t K, void* out, hipStream_t stream) {
  const int64_t nblocks = (N + 15) / 16;
  char cfg = M > 32 ? 'F' : (M <= 16 && nblocks < 512 ? 'B' : 'A');
  if (const char* env = getenv("CONVROT_W4A16_CFG"))
    if (env[0] == 'A' || env[0] == 'B' || env[0] == 'F') cfg = env[0];
  switch (cfg) {
    case 'A': return launch_t<ADT, ODT, 1, 2, 8, 3>(act, wq, ws, bias, M, N, K, out, stream);
    case 'B': return launch_t<ADT, ODT, 1, 1, 16, 4>(act, wq, ws, bias, M, N, K, out, stream);
    default: return launch_t<ADT, ODT, 4, 2, 4, 2>(act, wq, ws, bias, M, N, K, out, stream);
  }
}

template <int ADT>
hipError_t launch_odt(int odt, const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                      int64_t N, int64_t K, void* out, hipStream_t stream) {
  switch (odt) {
    case kF32: return launch_shape<ADT, kF32>(act, wq, ws, bias, M, N, K, out, stream);
    case kF16: return launch_shape<ADT, kF16>(act, wq, ws, bias, M, N, K, out, stream);
    default: return launch_shape<ADT, kBF16>(act, wq, ws, bias, M, N, K, out, stream);
  }
}

}  // namespace

hipError_t launch_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                             const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                             hipStream_t stream) {
  if (M == 0 || N == 0) return hipSuccess;
  if (act_dtype == kF16) return launch_odt<kF16>(out_dtype, act, qweight, wscales, bias, M, N, K, out, stream);
  return launch_odt<kBF16>(out_dtype, act, qweight, wscales, bias, M, N, K, out, stream);
}

}  // namespace convrot
