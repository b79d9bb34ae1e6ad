// Packed-int4 layout kernels for gfx950: pack, unpack and lossless weight
// re-layout between the reference's NK / KN layouts and the CDNA4 tile layout.
//
// These are HBM-bound byte permutations: one thread per output byte (or per
// four output bytes where rows allow), each gathering its two source nibbles.
// Reference counterparts: pack_signed_int4 / unpack_signed_int4
// (/root/reference/src/convrot_mlx/core.py:97-120), the Metal unpack kernel
// (:915-922), repack_nk_weight_for_mpp / repack_mpp_weight_to_nk (:123-146).
#include "convrot_device.h"
#include "convrot_launch.h"

namespace convrot {
namespace {

// pack: out[r, c] = (v[r, 2c] & 0xf) | ((v[r, 2c+1] & 0xf) << 4)   (core.py:101-105)
__global__ void pack_kernel(const int8_t* __restrict__ v, uint8_t* __restrict__ out, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint16_t pair = *(const uint16_t*)(v + 2 * i);
  out[i] = (uint8_t)((pair & 0x0fu) | ((pair >> 4) & 0xf0u));
}

// unpack: two's-complement nibbles -> int8 in [-8, 7], low nibble first (core.py:108-120, :919-921)
__global__ void unpack_kernel(const uint8_t* __restrict__ packed, int8_t* __restrict__ out, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint32_t b = packed[i];
  const int lo = (int)((b & 0x0fu) ^ 0x08u) - 8;
  const int hi = (int)((b >> 4) ^ 0x08u) - 8;
  *(uint16_t*)(out + 2 * i) = (uint16_t)((uint8_t)lo | ((uint32_t)(uint8_t)hi << 8));
}

// Four packed bytes -> eight int8 (two words), low nibble first.  Each nibble
// n becomes n | 0xf0 where its bit 3 is set: m = bit 3 of every byte, and
// m * 0xf0 sets the high half of exactly those bytes (no carries).
__device__ __forceinline__ uint2 unpack_word(uint32_t w) {
  uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  lo |= ((lo & 0x08080808u) >> 3) * 0xf0u;
  hi |= ((hi & 0x08080808u) >> 3) * 0xf0u;
  // interleave: bytes (lo0 hi0 lo1 hi1) and (lo2 hi2 lo3 hi3)
  return make_uint2(__builtin_amdgcn_perm(hi, lo, 0x05010400u), __builtin_amdgcn_perm(hi, lo, 0x07030602u));
}

// The same 16 packed bytes per thread: one 16-byte load, two 16-byte stores.
// Needs total % 16 == 0 and 16-byte aligned buffers (checked by the launcher).
__global__ void unpack16_kernel(const uint4* __restrict__ packed, uint4* __restrict__ out, int64_t vecs) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= vecs) return;
  const uint4 p = packed[i];
  const uint2 a = unpack_word(p.x), b = unpack_word(p.y), c = unpack_word(p.z), d = unpack_word(p.w);
  out[2 * i] = make_uint4(a.x, a.y, b.x, b.y);
  out[2 * i + 1] = make_uint4(c.x, c.y, d.x, d.y);
}

// Nibble (two's complement, 4 bits) of weight element (n, k) in a layout;
// zero outside the N x K weight (CDNA4 padding).
__device__ __forceinline__ uint32_t nibble_at(const uint8_t* __restrict__ in, int layout, int64_t n, int64_t k,
                                              int64_t N, int64_t K, int64_t nblocks) {
  if (n >= N || k >= K) return 0u;
  uint32_t byte;
  int shift;
  if (layout == CONVROT_LAYOUT_NK) {
    byte = in[n * (K >> 1) + (k >> 1)];
    shift = (int)(k & 1) * 4;
  } else if (layout == CONVROT_LAYOUT_KN) {
    byte = in[k * (N >> 1) + (n >> 1)];
    shift = (int)(n & 1) * 4;
  } else {
    const int64_t kb = k >> 7, nb = n >> 4;
    const int kk = (int)(k & 127), r = (int)(n & 15);
    const int q = kk >> 5, c = (kk >> 3) & 3, j = kk & 3, h = (kk >> 2) & 1;
    byte = in[(kb * nblocks + nb) * 1024 + (16 * q + r) * 16 + 4 * c + j];
    shift = h * 4;
  }
  return (byte >> shift) & 0x0fu;
}

// One output byte per thread: decode which two (n, k) elements it holds in the
// output layout, gather both nibbles from the input layout.
__global__ void repack_kernel(const uint8_t* __restrict__ in, int in_layout, uint8_t* __restrict__ out,
                              int out_layout, int64_t N, int64_t K, int64_t total, int64_t nblocks) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  int64_t n0, k0, n1, k1;
  if (out_layout == CONVROT_LAYOUT_NK) {
    const int64_t pk = K >> 1;
    n0 = n1 = i / pk;
    k0 = 2 * (i % pk);
    k1 = k0 + 1;
  } else if (out_layout == CONVROT_LAYOUT_KN) {
    const int64_t pn = N >> 1;
    k0 = k1 = i / pn;
    n0 = 2 * (i % pn);
    n1 = n0 + 1;
  } else {
    const int64_t blk = i >> 10;
    const int off = (int)(i & 1023);
    const int64_t kb = blk / nblocks, nb = blk % nblocks;
    const int L = off >> 4, c = (off >> 2) & 3, j = off & 3;
    const int q = L >> 4, r = L & 15;
    n0 = n1 = nb * 16 + r;
    k0 = kb * 128 + 32 * q + 8 * c + j;
    k1 = k0 + 4;
  }
  const uint32_t lo = nibble_at(in, in_layout, n0, k0, N, K, nblocks);
  const uint32_t hi = nibble_at(in, in_layout, n1, k1, N, K, nblocks);
  out[i] = (uint8_t)(lo | (hi << 4));
}

// FP6 fields of two's-complement nibbles, one byte per nibble value: 0 .. 7
// and (indexed by n & 7) 8 .. 15, i.e. -8 .. -1.  A code v is the e2m3
// encoding of v/8: the sign-magnitude subnormal for |v| <= 7, and -1.0
// (0x28) for -8.
constexpr uint64_t kFp6Pos = 0x0706050403020100ull;  // 0, 1 .. 7
constexpr uint64_t kFp6Neg = 0x2122232425262728ull;  // -8, -7 .. -1

// CDNA4 int4 weight -> FP6 operand blocks, one thread per 16-byte lane L of a
// 1024-byte CDNA4 block: its 32 nibbles (features 32 q + 8 c + j + 4 h at
// dword c, byte j, half h) become the lane's 24-byte FP6 stream (feature i at
// bits 6 i), head at 16 L and tail at 1024 + 8 L of the 1536-byte FP6 block.
__global__ void fp6_weight_kernel(const uint4* __restrict__ in, uint8_t* __restrict__ out, int64_t lanes) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= lanes) return;
  const uint4 v = in[t];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint64_t s[3] = {0, 0, 0};
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t n = (w[c] >> (8 * j + 4 * h)) & 15u;
        const uint64_t code = (((n & 8u) ? kFp6Neg : kFp6Pos) >> (8 * (n & 7u))) & 0x3fu;
        const int bit = 6 * (8 * c + 4 * h + j);
        s[bit >> 6] |= code << (bit & 63);
        if ((bit & 63) > 58) s[(bit >> 6) + 1] |= code >> (64 - (bit & 63));
      }
  uint8_t* o = out + (t >> 6) * 1536;
  const int L = (int)(t & 63);
  *(uint4*)(o + 16 * L) = make_uint4((uint32_t)s[0], (uint32_t)(s[0] >> 32), (uint32_t)s[1], (uint32_t)(s[1] >> 32));
  *(uint2*)(o + 1024 + 8 * L) = make_uint2((uint32_t)s[2], (uint32_t)(s[2] >> 32));
}

// CDNA4 int4 weight -> compact FP6 blocks (the FP6 stream of each lane with the
// two exponent bits of every field dropped: 1024 bytes a block, see
// fp6c_expand in gemm_w4a4.hip), one thread per 16-byte lane.  A code of -8
// (-1.0, the one field with an exponent) has no compact form: the lane stores
// its fields regardless and raises *minus8.
constexpr uint32_t kFp6cZ0 = 0x18618618u, kFp6cZ1 = 0x86186186u;

__global__ void fp6c_weight_kernel(const uint4* __restrict__ in, uint4* __restrict__ out, int* __restrict__ minus8,
                                   int64_t lanes) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= lanes) return;
  const uint4 v = in[t];
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint64_t s[3] = {0, 0, 0};
  bool bad = false;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t n = (w[c] >> (8 * j + 4 * h)) & 15u;
        bad |= n == 8u;
        const uint64_t code = (((n & 8u) ? kFp6Neg : kFp6Pos) >> (8 * (n & 7u))) & 0x3fu;
        const int bit = 6 * (8 * c + 4 * h + j);
        s[bit >> 6] |= code << (bit & 63);
        if ((bit & 63) > 58) s[(bit >> 6) + 1] |= code >> (64 - (bit & 63));
      }
  const uint32_t d0 = (uint32_t)s[0], d1 = (uint32_t)(s[0] >> 32), d2 = (uint32_t)s[1];
  const uint32_t d3 = (uint32_t)(s[1] >> 32), d4 = (uint32_t)s[2], d5 = (uint32_t)(s[2] >> 32);
  out[t] = make_uint4((d0 & ~kFp6cZ0) | (d2 & kFp6cZ0), (d1 & ~kFp6cZ1) | (d2 & kFp6cZ1),
                      (d3 & ~kFp6cZ0) | (d5 & kFp6cZ0), (d4 & ~kFp6cZ1) | (d5 & kFp6cZ1));
  if (bad && minus8) *minus8 = 1;
}

__global__ void zero_int_kernel(int* __restrict__ p) {
  if (threadIdx.x == 0) *p = 0;
}

inline unsigned grid_for(int64_t total, int block) { return (unsigned)((total + block - 1) / block); }

}  // namespace

hipError_t launch_pack_int4(const int8_t* values, int64_t rows, int64_t packed_cols, uint8_t* out,
                            hipStream_t stream) {
  const int64_t total = rows * packed_cols;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(pack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream, values, out, total);
  return hipGetLastError();
}

hipError_t launch_unpack_int4(const uint8_t* packed, int64_t rows, int64_t packed_cols, int8_t* out,
                              hipStream_t stream) {
  const int64_t total = rows * packed_cols;
  if (total == 0) return hipSuccess;
  if (total % 16 == 0 && (uintptr_t)packed % 16 == 0 && (uintptr_t)out % 16 == 0) {
    const int64_t vecs = total / 16;
    hipLaunchKernelGGL(unpack16_kernel, dim3(grid_for(vecs, 256)), dim3(256), 0, stream, (const uint4*)packed,
                       (uint4*)out, vecs);
  } else {
    hipLaunchKernelGGL(unpack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream, packed, out, total);
  }
  return hipGetLastError();
}

hipError_t launch_repack(const uint8_t* in, int in_layout, uint8_t* out, int out_layout, int64_t N, int64_t K,
                         hipStream_t stream) {
  const int64_t nblocks = (N + 15) / 16, kblocks = (K + 127) / 128;
  int64_t total;
  if (out_layout == CONVROT_LAYOUT_NK) total = N * (K / 2);
  else if (out_layout == CONVROT_LAYOUT_KN) total = K * (N / 2);
  else total = kblocks * nblocks * 1024;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(repack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream, in, in_layout, out,
                     out_layout, N, K, total, nblocks);
  return hipGetLastError();
}

hipError_t launch_weight_fp6c(const uint8_t* cdna4, uint8_t* fp6c, int* minus8, int64_t N, int64_t K,
                              hipStream_t stream) {
  const int64_t lanes = ((K + 127) / 128) * ((N + 15) / 16) * 64;
  if (minus8) {
    hipLaunchKernelGGL(zero_int_kernel, dim3(1), dim3(64), 0, stream, minus8);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
  }
  if (lanes == 0) return hipSuccess;
  hipLaunchKernelGGL(fp6c_weight_kernel, dim3(grid_for(lanes, 256)), dim3(256), 0, stream, (const uint4*)cdna4,
                     (uint4*)fp6c, minus8, lanes);
  return hipGetLastError();
}

hipError_t launch_weight_fp6(const uint8_t* cdna4, uint8_t* fp6, int64_t N, int64_t K, hipStream_t stream) {
  const int64_t lanes = ((K + 127) / 128) * ((N + 15) / 16) * 64;
  if (lanes == 0) return hipSuccess;
  hipLaunchKernelGGL(fp6_weight_kernel, dim3(grid_for(lanes, 256)), dim3(256), 0, stream, (const uint4*)cdna4, fp6,
                     lanes);
  return hipGetLastError();
}

}  // namespace convrot
