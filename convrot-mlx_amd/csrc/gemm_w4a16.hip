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
// of 16*FM tokens; its SPLIT waves stride over the 128-feature blocks of K and
// their partial sums are reduced through LDS in a fixed order (deterministic).
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

template <int ADT, int ODT, int FM, int NB, int SPLIT>
__global__ __launch_bounds__(SPLIT * 64) void w4a16_gemm_kernel(const uint16_t* __restrict__ act,
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

  for (int kb = wave; kb < kblocks; kb += SPLIT) {
    // activation operands: lane (m = r, q) -> 8 values at features kb*128 + 32q + 8c
    i32x4 aop[FM][4];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = m0 + fm * 16 + r;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int k = kb * 128 + 32 * q + 8 * c;
        aop[fm][c] = (m < M && k < K) ? *(const i32x4*)(act + (int64_t)m * K + k) : (i32x4){0, 0, 0, 0};
      }
    }
    uint4 w[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const int nb = nb0 + t;
      w[t] = nb < nblocks ? *(const uint4*)(wq + ((int64_t)kb * nblocks + nb) * 1024 + lane * 16)
                          : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const uint32_t wd[4] = {w[t].x, w[t].y, w[t].z, w[t].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const i32x4 bop = expand8<ADT>(wd[c]);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) acc[t][fm] = mfma16<ADT>(bop, aop[fm][c], acc[t][fm]);
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

template <int ADT, int ODT, int FM, int NB, int SPLIT>
hipError_t launch_t(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M, int64_t N,
                    int64_t K, void* out, hipStream_t stream) {
  const int nblocks = (int)((N + 15) / 16), kblocks = (int)((K + 127) / 128);
  dim3 grid((unsigned)((nblocks + NB - 1) / NB), (unsigned)((M + 16 * FM - 1) / (16 * FM)));
  hipLaunchKernelGGL((w4a16_gemm_kernel<ADT, ODT, FM, NB, SPLIT>), grid, dim3(64 * SPLIT), 0, stream,
                     (const uint16_t*)act, wq, ws, bias, out, (int)M, (int)N, (int)K, nblocks, kblocks);
  return hipGetLastError();
}

template <int ADT, int ODT>
hipError_t launch_shape(const void* act, const uint8_t* wq, const float* ws, const float* bias, int64_t M,
                        int64_t N, int64_t K, void* out, hipStream_t stream) {
  const int64_t kblocks = (K + 127) / 128;
  // split K across waves when there are few weight tiles per token tile
  const bool deep = kblocks >= 32;
  if (M <= 16) {
    return deep ? launch_t<ADT, ODT, 1, 2, 8>(act, wq, ws, bias, M, N, K, out, stream)
                : launch_t<ADT, ODT, 1, 2, 4>(act, wq, ws, bias, M, N, K, out, stream);
  }
  if (M <= 32) {
    return deep ? launch_t<ADT, ODT, 2, 2, 8>(act, wq, ws, bias, M, N, K, out, stream)
                : launch_t<ADT, ODT, 2, 2, 4>(act, wq, ws, bias, M, N, K, out, stream);
  }
  return launch_t<ADT, ODT, 4, 2, 4>(act, wq, ws, bias, M, N, K, out, stream);
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
