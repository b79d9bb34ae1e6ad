// Fused ConvRot activation preparation for gfx950: normalized regular-Hadamard
// rotation + rowwise absmax + symmetric A4 quantization + packing, one pass.
//
// Replaces the reference's two-pass Metal kernels (one threadgroup per row,
// a barrier per butterfly stage, the row read and rotated twice:
// /root/reference/src/convrot_mlx/core.py:205-304 packed, :307-327 int8,
// :330-370 rotate-only) and reproduces the eager contract bit for bit
// (regular_hadamard core.py:64-94, quantize_signed_int4_rowwise :149-158).
//
// Data layout and work split
//  * One workgroup per row, W waves per row, NI iterations per wave.  In one
//    iteration a wave owns 1024 consecutive features: lane l holds the 16
//    consecutive features [16l, 16l+16) in registers (two 16-byte loads).
//  * A feature index inside a group of G = 4^S is written in base 4 as
//    (d_{S-1} ... d1 d0).  Stage s of the butterfly runs along digit d_s
//    (stride 4^s).  Phase 1 keeps (d1, d0) in registers and runs stages 0
//    and 1 without any data movement; every later stage s keeps (d_s, d0) in
//    registers and is reached through one LDS exchange (four 16-byte writes,
//    four 16-byte reads per lane, wave-private region, no workgroup barrier).
//  * The rotated row stays in registers (NI*16 floats per lane) until the
//    row absmax is known -- one HBM read of x instead of the reference's two.
//  * bf16 rounding after every add costs one v_cvt_pk_bf16_f32 (see
//    round_bf16); the division by scale is a multiply by a correctly rounded
//    reciprocal, which is exact for bf16 operands (r/scale can never lie
//    within 2^-16.8 of a bf16 rounding midpoint, so an error below 2^-23
//    cannot change the rounded ratio).  f16/f32 inputs use a true division.
#include <stdlib.h>

#include "convrot_device.h"
#include "convrot_launch.h"

namespace convrot {
namespace {

constexpr int kMaxWaves = 16;
constexpr int kMaxBlocks = 64;  // 1024-feature blocks of the longest row (65536 features)
constexpr int kRegionFloats = 1280;  // per wave: 1024 features + 1/4 padding

// One radix-4 butterfly with a dtype rounding after every add (core.py:89-91):
//   a+b+c-d, a+b-c+d, a-b+c+d, -a+b+c+d, each evaluated left to right.
// rnd(-a+b) == -rnd(a-b) exactly, so the fourth output reuses a-b.
template <int DT>
__device__ __forceinline__ void radix4(float& a, float& b, float& c, float& d) {
  const float t1 = rnd<DT>(a + b);
  const float t2 = rnd<DT>(a - b);
  const float u0 = rnd<DT>(t1 + c);
  const float u1 = rnd<DT>(t1 - c);
  const float u2 = rnd<DT>(t2 + c);
  const float u3 = rnd<DT>(c - t2);
  a = rnd<DT>(u0 - d);
  b = rnd<DT>(u1 + d);
  c = rnd<DT>(u2 + d);
  d = rnd<DT>(u3 + d);
}

// Stage along d0 (register slots 4r .. 4r+3).
template <int DT>
__device__ __forceinline__ void stage_lo(float (&v)[16]) {
#pragma unroll
  for (int r = 0; r < 4; ++r) radix4<DT>(v[4 * r], v[4 * r + 1], v[4 * r + 2], v[4 * r + 3]);
}

// Stage along the digit held in register-slot bits 2-3.
template <int DT>
__device__ __forceinline__ void stage_hi(float (&v)[16]) {
#pragma unroll
  for (int d0 = 0; d0 < 4; ++d0) radix4<DT>(v[d0], v[4 + d0], v[8 + d0], v[12 + d0]);
}

// Index inside the group of register run `run` (slots 4*run .. 4*run+3,
// digit d0 = 0..3) for a lane at position p of its group during phase PH.
// Phase 1: (d1, d0) in registers, the lane owns features 16p .. 16p+15.
// Phase PH >= 2: (d_PH, d0) in registers, the remaining digits
// d1..d_{S-1} (skipping d_PH) come from p, lowest first.
template <int S, int PH>
__device__ __forceinline__ int run_index(int p, int run) {
  if constexpr (PH == 1) {
    return 16 * p + 4 * run;
  } else {
    int i = 0, pp = p, w = 4;
#pragma unroll
    for (int t = 1; t < S; ++t, w *= 4) {
      int digit;
      if (t == PH) {
        digit = run;
      } else {
        digit = pp & 3;
        pp >>= 2;
      }
      i += digit * w;
    }
    return i;
  }
}

// Padded LDS offset (floats): 4 floats of padding after every 16 features,
// which keeps the phase-1 writes and the phase-2 reads bank-conflict free.
__device__ __forceinline__ int lds_off(int i) { return i + 4 * (i >> 4); }

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Move the lane's 16 values from the phase PH-1 layout to the phase PH layout
// through the wave's LDS region and run stage PH.
template <int DT, int S, int PH>
__device__ __forceinline__ void exchange_and_stage(float (&v)[16], float* region, int p) {
#pragma unroll
  for (int run = 0; run < 4; ++run) {
    const int i = run_index<S, PH - 1>(p, run);
    *(float4*)(region + lds_off(i)) = make_float4(v[4 * run], v[4 * run + 1], v[4 * run + 2], v[4 * run + 3]);
  }
  wave_lds_fence();
#pragma unroll
  for (int run = 0; run < 4; ++run) {
    const int i = run_index<S, PH>(p, run);
    const float4 t = *(const float4*)(region + lds_off(i));
    v[4 * run] = t.x;
    v[4 * run + 1] = t.y;
    v[4 * run + 2] = t.z;
    v[4 * run + 3] = t.w;
  }
  wave_lds_fence();
  stage_hi<DT>(v);
}

template <int DT, int S>
__device__ __forceinline__ void rotate16(float (&v)[16], float* region, int p) {
  if constexpr (S >= 1) stage_lo<DT>(v);
  if constexpr (S >= 2) stage_hi<DT>(v);
  if constexpr (S >= 3) exchange_and_stage<DT, S, 2>(v, region, p);
  if constexpr (S >= 4) exchange_and_stage<DT, S, 3>(v, region, p);
  if constexpr (S >= 5) exchange_and_stage<DT, S, 4>(v, region, p);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// 16 consecutive elements at byte `off` of the row's buffer (16-byte loads);
// offsets at or beyond the row's end read as zero (buffer range check).
template <int DT>
__device__ __forceinline__ void load16(__amdgpu_buffer_rsrc_t row, uint32_t off, float (&v)[16]) {
  if constexpr (DT == kF32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u32x4 t = __builtin_amdgcn_raw_buffer_load_b128(row, (int)(off + 16 * q), 0, 0);
      // __uint_as_float, not __builtin_bit_cast: this compiler bit_casts a
      // vector-element operand from element 0's storage
      v[4 * q] = __uint_as_float(t.x);
      v[4 * q + 1] = __uint_as_float(t.y);
      v[4 * q + 2] = __uint_as_float(t.z);
      v[4 * q + 3] = __uint_as_float(t.w);
    }
  } else {
    const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(row, (int)off, 0, 0);
    const u32x4 b = __builtin_amdgcn_raw_buffer_load_b128(row, (int)(off + 16), 0, 0);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if constexpr (DT == kBF16) {
        v[2 * q] = bf16_lo(w[q]);
        v[2 * q + 1] = bf16_hi(w[q]);
      } else {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        const f16x2 h = __builtin_bit_cast(f16x2, w[q]);
        v[2 * q] = (float)h[0];
        v[2 * q + 1] = (float)h[1];
      }
    }
  }
}

// max(m, |a|, |b|) in one v_max3_f32 with |.| source modifiers (m >= 0).  As
// C++ the compiler inserts canonicalizing moves and separate abs masks.
__device__ __forceinline__ float absmax3(float m, float a, float b) {
  float r;
  asm("v_max3_f32 %0, |%1|, |%2|, %3" : "=v"(r) : "v"(a), "v"(b), "v"(m));
  return r;
}

// Maximum over the wave of a non-negative float (bit patterns of non-negative
// floats order like unsigned integers): DPP quad swaps and row mirrors leave
// every lane of a 16-lane row with the row maximum, then four readlanes.
__device__ __forceinline__ float wave_max_nonneg(float x) {
  uint32_t v = __builtin_bit_cast(uint32_t, x);
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));   // quad_perm [1,0,3,2]
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));   // quad_perm [2,3,0,1]
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, true));  // row_half_mirror
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, true));  // row_mirror
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
  const uint32_t r1 = (uint32_t)__builtin_amdgcn_readlane((int)v, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)v, 32);
  const uint32_t r3 = (uint32_t)__builtin_amdgcn_readlane((int)v, 48);
  return __builtin_bit_cast(float, max(max(r0, r1), max(r2, r3)));
}

// Signed code in [-7, 7] of a ratio: clamp, then round half to even by adding
// 1.5 * 2^23 (the float add rounds to the nearest integer, ties to even, and
// leaves the integer in the low mantissa bits in two's complement).
__device__ __forceinline__ uint32_t code_bits(float ratio) {
  const float c = __builtin_amdgcn_fmed3f(ratio, -7.0f, 7.0f);
  return __builtin_bit_cast(uint32_t, c + 12582912.0f);
}

// Four codes (low bytes of code_bits) gathered into one int8x4 word.
__device__ __forceinline__ uint32_t gather_bytes(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t lo = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm(b3, b2, 0x04000c0cu);
  return lo | hi;
}

// Four codes packed as four nibbles, low nibble = lowest feature (core.py:101-105).
__device__ __forceinline__ uint32_t gather_nibbles(uint32_t b0, uint32_t b1, uint32_t b2, uint32_t b3) {
  const uint32_t bytes = gather_bytes(b0, b1, b2, b3) & 0x0f0f0f0fu;
  const uint32_t pairs = bytes | (bytes >> 4);  // byte0 = n0|n1<<4, byte2 = n2|n3<<4
  return __builtin_amdgcn_perm(0u, pairs, 0x0c0c0200u);
}

// FP6 operand codes.  A code v is stored as the e2m3 encoding of v/8: for
// |v| <= 7 that is the subnormal with mantissa |v| (sign bit 5, exponent bits
// 4..3 zero), so the field is the sign-magnitude form of v; the GEMM's MFMA
// scales both operands by 2^3 and sums the exact products v*w.  Zero codes
// are +0.
//
// Four A4 codes as FP6 fields, packed as a 24-bit field (code j at bits
// 6j..6j+5).  m0..m3 are code_bits of the ratios' magnitudes (low byte |q| in
// 0..7) and r0..r3 the ratios, whose signs pick the negative codes.
__device__ __forceinline__ uint32_t fp6_piece(uint32_t m0, uint32_t m1, uint32_t m2, uint32_t m3, float r0, float r1,
                                              float r2, float r3) {
  const uint32_t mag = gather_bytes(m0, m1, m2, m3);
  const uint32_t pos = mag;                                                    // 0 .. 7
  const uint32_t neg = __builtin_amdgcn_perm(0x27262524u, 0x23222100u, mag);  // 0, -1 .. -7
  // selector 9 / 11: the sign bit of the second / first operand, over the byte
  const uint32_t sm = __builtin_amdgcn_perm(__float_as_uint(r1), __float_as_uint(r0), 0x0c0c0b09u) |
                      __builtin_amdgcn_perm(__float_as_uint(r3), __float_as_uint(r2), 0x0b090c0cu);
  const uint32_t codes = (neg & sm) | (pos & ~sm);
  const uint32_t y = (codes & 0x003f003fu) | ((codes >> 2) & 0x0fc00fc0u);  // 12-bit pairs at bits 0, 16
  return (y & 0xfffu) | ((y >> 4) & 0xfff000u);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x32 __attribute__((ext_vector_type(32)));
typedef int i32x6 __attribute__((ext_vector_type(6)));

// A pair of bf16 ratios with the sign cleared on each negative one of
// magnitude at most 0.5 (bits 0x3f00), i.e. on each ratio whose code
// rint(ratio) is 0: bit 15 of h + 0x40ff (per half, mod 2^16) is set for
// exactly those negative halves (and for positive halves above 0.5, whose
// sign bit is already clear).
__device__ __forceinline__ uint32_t zero_code_sign_fix(uint32_t h) {
  const u16x2 s = __builtin_bit_cast(u16x2, h) + (u16x2){0x40ff, 0x40ff};
  return h & ~(__builtin_bit_cast(uint32_t, s) & 0x80008000u);
}

// FP6 fields of 16 bf16 ratios (8 packed pairs, lowest feature first), whose
// magnitudes are at most 7.04 (as every bf16 ratio is, the scale being
// bf16(absmax / 7)): v_cvt_scalef32_pk32_fp6_bf16 divides by the scale 8 and
// rounds to the e2m3 grid of eighths with ties to even, so field i is
// rint(ratio_i) / 8 -- the code with its sign -- and fields 0..15 fill the
// first 96 bits (the other 16 inputs are zero).
__device__ __forceinline__ void fp6_fields16(const uint32_t (&hp)[8], uint32_t& d0, uint32_t& d1, uint32_t& d2) {
  const u32x16 in = {hp[0], hp[1], hp[2], hp[3], hp[4], hp[5], hp[6], hp[7], 0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  const i32x6 f = __builtin_amdgcn_cvt_scalef32_pk32_fp6_bf16(__builtin_bit_cast(bf16x32, in), 8.0f);
  d0 = (uint32_t)f[0];
  d1 = (uint32_t)f[1];
  d2 = (uint32_t)f[2];
}

// Sum of a float64 over the wave (butterfly: every lane ends with the total,
// added in the same order in every lane).
__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  return v;
}

// tanh GELU of the fused GELU producer, float32, in this fixed sequence (the
// same IEEE operations, in the same order, as the CPU oracle's gelu_tanh32):
//   x3 = (x * x) * x;  u = kBeta * fma(kKappa, x3, x)
//   q = 2 / (exp(2|u|) + 1)  (0 where 2|u| > 88 or u is NaN)
//   1 + tanh(u) = u >= 0 ? 2 - q : q  (no cancellation on either side)
//   y = (0.5 * x) * (1 + tanh(u))
// with exp(z) = 2^n e^r, n = rint(z log2 e), r = z - n ln2 by two fmas
// (Cody-Waite), e^r by its degree-7 Taylor polynomial (Horner, fma).
__device__ __forceinline__ float gelu_tanh32(float x) {
  const float x3 = (x * x) * x;
  const float u = 0x1.988454p-1f * __builtin_fmaf(0x1.6e4e26p-5f, x3, x);
  const float z = fabsf(u) + fabsf(u);
  float q = 0.0f;
  if (z <= 88.0f) {
    const float n = rintf(z * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, z);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1p-1f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    q = 2.0f / (ldexpf(p, (int)n) + 1.0f);
  }
  const float onept = u >= 0.0f ? 2.0f - q : q;
  return (0.5f * x) * onept;
}

// Producers: what the preparation reads as its input rows.
enum Producer : int {
  kProPlain = 0,     // x
  kProModulate = 1,  // (1 + scale) * layer_norm(x) + shift
  kProGelu = 2,      // [head | gelu_tanh(x)], each with its own row stride
};

// Arguments of the producers beyond x (unused fields are ignored).
struct ProducerArgs {
  const void* shift;  // kProModulate: [vectors, K] shift and scale rows
  const void* scale;
  int rows_per_vector;
  float eps;
  const void* head;     // kProGelu: [rows, head_features] at head_stride elements per row
  int head_features;    //   (0: no head), a multiple of 16
  int64_t head_stride;
  int64_t x_stride;     // kProGelu: elements per row of x (x has K - head_features features)
};

// PRO = kProModulate: the fused modulated producer.  Each row is first replaced by
//   y = rb(rb(rb(1 + scale) * rb((x - mean) * rstd)) + shift)
// (LayerNorm without affine parameters, then the adaLN modulation with a
// dtype rounding after every op), with the shift / scale row
// v = row / rows_per_vector.  Then the ConvRot preparation runs on y as it
// would on x.  The moments are float64 sums in a fixed order that does not
// depend on the launch plan: lane l of 1024-feature block b adds features
// 16l .. 16l+15 in order, the 64 lanes are combined by the xor butterfly of
// wave_sum_f64, and the block sums are added in block order.
//
// PRO = kProGelu: the fused GELU producer.  Feature f of a row is head[f] for
// f < head_features and rb(gelu_tanh32(x[f - head_features])) after that;
// padding past K reads zeros, and gelu(0) = 0.
template <int DT, int S, int NI, int MODE, int PRO>
__global__ __launch_bounds__(1024) void prep_kernel(const void* __restrict__ x, void* __restrict__ out,
                                                     float* __restrict__ scales, int K, ProducerArgs pa) {
  constexpr bool PRE = PRO == kProModulate;
  extern __shared__ float lds[];
  __shared__ float wave_max[kMaxWaves];
  __shared__ double block_moments[PRE ? kMaxBlocks : 1][2];

  constexpr int G = (S == 0) ? 1 : (1 << (2 * S));
  constexpr int LG = (S >= 3) ? (G / 16) : 1;        // lanes per group
  constexpr int GS = (S >= 3) ? G : 16;               // features per lane group
  constexpr bool kImplicitNorm = (DT == kBF16);      // x/sqrt(G) is exact in bf16
  constexpr float kNorm = (S == 0) ? 1.0f : 1.0f / (float)(1 << S);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  int64_t row = blockIdx.x;
  if constexpr (MODE == CONVROT_PREP_FP6) {
    // Workgroups go round-robin to the 8 XCDs.  The 16 rows of an FP6 block
    // share its cache lines, so each XCD takes runs of consecutive rows (a
    // multiple of 16 each) and its L2 merges the rows' pieces of a line.
    const int64_t run = ((int64_t)gridDim.x / (8 * 16)) * 16;
    if (row < 8 * run) row = (row & 7) * run + (row >> 3);
  }
  const int chunks = K >> 4;
  constexpr int kEsize = DT == kF32 ? 4 : 2;
  const __amdgpu_buffer_rsrc_t xrow = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const char*)x + row * (PRO == kProGelu ? pa.x_stride : (int64_t)K) * kEsize), (short)0,
      (PRO == kProGelu ? K - pa.head_features : K) * kEsize, 0x00020000);
  const __amdgpu_buffer_rsrc_t hrow = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(PRO == kProGelu && pa.head_features ? (const char*)pa.head + row * pa.head_stride * kEsize
                                                  : (const char*)x),
      (short)0, PRO == kProGelu ? pa.head_features * kEsize : 0, 0x00020000);
  float* region = lds + wave * kRegionFloats + (lane / LG) * (G + G / 4);
  const int p = lane % LG;

  float keep[NI][16];
  float amax = 0.0f;

  if constexpr (PRE) {
    const int real_blocks = (chunks + 63) >> 6;
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int block = wave * NI + it;
      load16<DT>(xrow, (uint32_t)(block * 64 + lane) * (16u * kEsize), keep[it]);  // past the row end: zeros
      double b1 = 0.0, b2 = 0.0;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const double d = (double)keep[it][j];
        b1 += d;
        b2 += d * d;
      }
      b1 = wave_sum_f64(b1);
      b2 = wave_sum_f64(b2);
      if (lane == 0 && block < real_blocks) {
        block_moments[block][0] = b1;
        block_moments[block][1] = b2;
      }
    }
    __syncthreads();
    double s1 = 0.0, s2 = 0.0;
    for (int b = 0; b < real_blocks; ++b) {
      s1 += block_moments[b][0];
      s2 += block_moments[b][1];
    }
    const double m64 = s1 / (double)K;
    double var = s2 / (double)K - m64 * m64;
    var = var > 0.0 ? var : 0.0;
    const float mean = (float)m64;
    const float rstd = (float)(1.0 / sqrt(var + (double)pa.eps));
    const int64_t vrow = row / pa.rows_per_vector;
    const __amdgpu_buffer_rsrc_t shrow = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)pa.shift + vrow * K * kEsize), (short)0, K * kEsize, 0x00020000);
    const __amdgpu_buffer_rsrc_t scrow = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)pa.scale + vrow * K * kEsize), (short)0, K * kEsize, 0x00020000);
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int chunk = (wave * NI + it) * 64 + lane;
      if (chunk >= chunks) continue;  // padding stays zero (whole groups lie past K)
      float sh[16], sc[16];
      load16<DT>(shrow, (uint32_t)chunk * (16u * kEsize), sh);
      load16<DT>(scrow, (uint32_t)chunk * (16u * kEsize), sc);
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        // The float32 product is rounded before the dtype rounding, as in the
        // eager graph: left to itself the compiler folds multiply-and-narrow
        // into one v_fma_mix (a single rounding of the exact product to f16),
        // which differs where the float32 product lands on an f16 midpoint.
        float prod = (keep[it][j] - mean) * rstd;
        asm volatile("" : "+v"(prod));
        const float ln = rnd<DT>(prod);
        keep[it][j] = rnd<DT>(rnd<DT>(rnd<DT>(1.0f + sc[j]) * ln) + sh[j]);
      }
    }
  }

  // FP6 output: every iteration's loads go out before the first rotation, so
  // the wave's whole share of the row is in flight at once (5 % faster at
  // 4608 x 15360, 1 % at K = 3072; the INT8 output ran 3-15 % slower so)
  constexpr bool kPrefetch = PRO == kProPlain && MODE == CONVROT_PREP_FP6;
  if constexpr (kPrefetch) {
#pragma unroll
    for (int it = 0; it < NI; ++it)
      load16<DT>(xrow, (uint32_t)((wave * NI + it) * 64 + lane) * (16u * kEsize), keep[it]);  // past the end: zeros
  }
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int block = wave * NI + it;
    const int chunk = block * 64 + lane;
    float (&v)[16] = keep[it];
    if constexpr (PRO == kProPlain && !kPrefetch) {
      load16<DT>(xrow, (uint32_t)chunk * (16u * kEsize), v);  // chunks past the row end read zeros
    } else if constexpr (PRO == kProGelu) {
      const int f0 = chunk * 16;  // head_features % 16 == 0: a chunk lies in one segment
      if (f0 < pa.head_features) {
        load16<DT>(hrow, (uint32_t)f0 * kEsize, v);
      } else {
        load16<DT>(xrow, (uint32_t)(f0 - pa.head_features) * kEsize, v);  // past the end: zeros
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          // the float32 result is rounded on its own, as the oracle does (no
          // multiply-and-narrow folding into one v_fma_mix for f16)
          float g = gelu_tanh32(v[j]);
          asm volatile("" : "+v"(g));
          v[j] = rnd<DT>(g);
        }
      }
    }
    rotate16<DT, S>(v, region, p);
    if constexpr (!kImplicitNorm && S > 0 && MODE != CONVROT_PREP_ROTATE) {
#pragma unroll
      for (int j = 0; j < 16; ++j) v[j] = rnd<DT>(v[j] * kNorm);
    }
    if constexpr (MODE != CONVROT_PREP_ROTATE) {
#pragma unroll
      for (int j = 0; j < 16; j += 2) amax = absmax3(amax, v[j], v[j + 1]);
    }
  }

  // ---- row scale (core.py:154-156)
  float inv = 0.0f, scale = 0.0f;
  if constexpr (MODE != CONVROT_PREP_ROTATE) {
    amax = wave_max_nonneg(amax);
    if (nwaves > 1) {
      if (lane == 0) wave_max[wave] = amax;
      __syncthreads();
      amax = wave_max[0];
      for (int w = 1; w < nwaves; ++w) amax = fmaxf(amax, wave_max[w]);
    }
    if constexpr (kImplicitNorm) amax *= kNorm;
    float floor_v;
    if constexpr (DT == kBF16) floor_v = __builtin_bit_cast(float, 0x2edc0000u);  // bf16(1e-10)
    else if constexpr (DT == kF16) floor_v = 0.0f;                                // f16(1e-10) underflows
    else floor_v = 1e-10f;
    scale = rnd<DT>(fmaxf(amax, floor_v) / 7.0f);
    if constexpr (kImplicitNorm) inv = (1.0f / scale) * kNorm;
    if (wave == 0 && lane == 0) scales[row] = scale;
  }

  // ---- quantize + store, phase-final layout
  constexpr int PHF = (S >= 3) ? (S - 1) : 1;
#pragma unroll
  for (int it = 0; it < NI; ++it) {
    const int block = wave * NI + it;
    const int chunk = block * 64 + lane;
    if (chunk >= chunks) continue;
    const int64_t gbase = row * K + (int64_t)block * 1024 + (lane / LG) * GS;
    const float (&v)[16] = keep[it];
    uint32_t q[16];
    float rt[16];
    constexpr bool kFp6Cvt = MODE == CONVROT_PREP_FP6 && DT == kBF16;  // FP6 by the conversion instruction
    if constexpr (MODE != CONVROT_PREP_ROTATE && !kFp6Cvt) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float ratio;
        if constexpr (DT == kBF16) ratio = round_bf16(v[j] * inv);
        else ratio = scale > 0.0f ? rnd<DT>(v[j] / scale) : 0.0f;  // 0/0 on an all-zero f16 row
        // FP6 keeps |q| and the ratio's sign (rint is symmetric: |rint(c)| = rint(|c|))
        q[j] = code_bits(MODE == CONVROT_PREP_FP6 ? fabsf(ratio) : ratio);
        rt[j] = ratio;
      }
    }
    if constexpr (MODE == CONVROT_PREP_FP6) {
      // 16 consecutive features (a group's half stream, 12 bytes) are 4 runs
      // of 4: the lane's own 4 runs for groups up to 16, else run r of the 4
      // lanes of a quad (lane k holding features 4k .. 4k+3 of it), which
      // lane r of the quad gathers through the wave's LDS region.
      uint32_t d0, d1, d2;
      int fh;  // first feature (in the row) of the half this lane writes
      const int qb = lane & ~3, k = lane & 3;
      uint32_t* xr = (uint32_t*)(lds + wave * kRegionFloats);
      if constexpr (kFp6Cvt) {
        // bf16 ratios, two to a register (run r in hp[2r], hp[2r+1]), then one
        // conversion instruction for the lane's 16 features
        uint32_t hp[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) hp[i] = zero_code_sign_fix(pack_bf16x2(v[2 * i] * inv, v[2 * i + 1] * inv));
        if constexpr (S >= 3) {
          wave_lds_fence();
#pragma unroll
          for (int run = 0; run < 4; ++run)
            *(uint2*)(xr + (qb + run) * 8 + 2 * k) = make_uint2(hp[2 * run], hp[2 * run + 1]);
          wave_lds_fence();
          const uint4 g0 = *(const uint4*)(xr + (qb + k) * 8), g1 = *(const uint4*)(xr + (qb + k) * 8 + 4);
          hp[0] = g0.x, hp[1] = g0.y, hp[2] = g0.z, hp[3] = g0.w;
          hp[4] = g1.x, hp[5] = g1.y, hp[6] = g1.z, hp[7] = g1.w;
        }
        fp6_fields16(hp, d0, d1, d2);
      } else {
        // each run's four codes as a 24-bit field
        uint32_t pc[4];
#pragma unroll
        for (int run = 0; run < 4; ++run)
          pc[run] = fp6_piece(q[4 * run], q[4 * run + 1], q[4 * run + 2], q[4 * run + 3], rt[4 * run],
                              rt[4 * run + 1], rt[4 * run + 2], rt[4 * run + 3]);
        if constexpr (S >= 3) {
          wave_lds_fence();
#pragma unroll
          for (int run = 0; run < 4; ++run) xr[(qb + run) * 4 + k] = pc[run];
          wave_lds_fence();
          const uint4 g = *(const uint4*)(xr + (qb + k) * 4);
          pc[0] = g.x, pc[1] = g.y, pc[2] = g.z, pc[3] = g.w;
        }
        d0 = pc[0] | (pc[1] << 24);
        d1 = (pc[1] >> 8) | (pc[2] << 16);
        d2 = (pc[2] >> 16) | (pc[3] << 8);
      }
      if constexpr (S >= 3) fh = block * 1024 + (lane / LG) * GS + run_index<S, PHF>(p & ~3, k);
      else fh = block * 1024 + lane * 16;
      const int64_t mblocks = ((int64_t)gridDim.x + 15) >> 4;
      uint8_t* blk = (uint8_t*)out + ((int64_t)(fh >> 7) * mblocks + (row >> 4)) * 1536;
      const int L = ((fh >> 5) & 3) * 16 + (int)(row & 15);
      // The two halves of a 32-feature group share slot L: 12 bytes of the
      // first, then the second's first dword (its other 8 bytes go to the
      // block's tail).  They sit in lanes kPair apart (bit 4 of fh is lane bit
      // 2 for groups of 256 and 1024, lane bit 0 otherwise), so the first lane
      // writes the whole 16-byte slot: two stores a pair instead of three.
      // Both lanes of a pair are past the row end or neither (K % 128 == 0).
      constexpr int kPair = (S == 4 || S == 5) ? 4 : 1;
      const uint32_t d0_second = (uint32_t)__shfl_down((int)d0, kPair);
      if ((fh & 16) == 0) {
        *(uint4*)(blk + 16 * L) = make_uint4(d0, d1, d2, d0_second);
      } else {
        *(uint2*)(blk + 1024 + 8 * L) = make_uint2(d1, d2);
      }
      continue;
    }
#pragma unroll
    for (int run = 0; run < 4; ++run) {
      const int64_t f = gbase + run_index<(S >= 3 ? S : 3), PHF>(p, run);
      const float* vr = &v[4 * run];
      if constexpr (MODE == CONVROT_PREP_INT8) {
        ((uint32_t*)out)[f >> 2] = gather_bytes(q[4 * run], q[4 * run + 1], q[4 * run + 2], q[4 * run + 3]);
      } else if constexpr (MODE == CONVROT_PREP_PACKED) {
        ((uint16_t*)out)[f >> 2] =
            (uint16_t)gather_nibbles(q[4 * run], q[4 * run + 1], q[4 * run + 2], q[4 * run + 3]);
      } else {
        // core.py:94 -- y / sqrt(G), rounded to the dtype
        store_out4<DT>(out, f, rnd<DT>(vr[0] * kNorm), rnd<DT>(vr[1] * kNorm), rnd<DT>(vr[2] * kNorm),
                       rnd<DT>(vr[3] * kNorm));
      }
    }
  }
}

// The producer of a launch and its arguments.
struct Modulation {
  int producer;  // kProPlain, kProModulate or kProGelu
  ProducerArgs args;
};

template <int DT, int S, int NI, int MODE>
hipError_t launch_prep_t(const void* x, void* out, float* scales, int64_t rows, int K, int waves,
                         const Modulation& mod, hipStream_t stream) {
  const size_t lds_bytes = (S >= 3) ? (size_t)waves * kRegionFloats * sizeof(float) : 0;
  if (mod.producer == kProModulate)
    hipLaunchKernelGGL((prep_kernel<DT, S, NI, MODE, kProModulate>), dim3((unsigned)rows), dim3(64 * waves),
                       lds_bytes, stream, x, out, scales, K, mod.args);
  else if (mod.producer == kProGelu)
    hipLaunchKernelGGL((prep_kernel<DT, S, NI, MODE, kProGelu>), dim3((unsigned)rows), dim3(64 * waves),
                       lds_bytes, stream, x, out, scales, K, mod.args);
  else
    hipLaunchKernelGGL((prep_kernel<DT, S, NI, MODE, kProPlain>), dim3((unsigned)rows), dim3(64 * waves),
                       lds_bytes, stream, x, out, scales, K, mod.args);
  return hipGetLastError();
}

template <int DT, int S, int NI>
hipError_t launch_prep_mode(int mode, const void* x, void* out, float* scales, int64_t rows, int K,
                            int waves, const Modulation& mod, hipStream_t stream) {
  switch (mode) {
    case CONVROT_PREP_PACKED:
      return launch_prep_t<DT, S, NI, CONVROT_PREP_PACKED>(x, out, scales, rows, K, waves, mod, stream);
    case CONVROT_PREP_FP6:
      return launch_prep_t<DT, S, NI, CONVROT_PREP_FP6>(x, out, scales, rows, K, waves, mod, stream);
    case CONVROT_PREP_INT8:
      return launch_prep_t<DT, S, NI, CONVROT_PREP_INT8>(x, out, scales, rows, K, waves, mod, stream);
    default: return launch_prep_t<DT, S, NI, CONVROT_PREP_ROTATE>(x, out, scales, rows, K, waves, mod, stream);
  }
}

template <int DT, int S>
hipError_t launch_prep_ni(int ni, int mode, const void* x, void* out, float* scales, int64_t rows, int K,
                          int waves, const Modulation& mod, hipStream_t stream) {
  switch (ni) {
    case 1: return launch_prep_mode<DT, S, 1>(mode, x, out, scales, rows, K, waves, mod, stream);
    case 3: return launch_prep_mode<DT, S, 3>(mode, x, out, scales, rows, K, waves, mod, stream);
    default: return launch_prep_mode<DT, S, 4>(mode, x, out, scales, rows, K, waves, mod, stream);
  }
}

template <int DT>
hipError_t launch_prep_s(int s, int ni, int mode, const void* x, void* out, float* scales, int64_t rows,
                         int K, int waves, const Modulation& mod, hipStream_t stream) {
  switch (s) {
    case 0: return launch_prep_ni<DT, 0>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
    case 1: return launch_prep_ni<DT, 1>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
    case 2: return launch_prep_ni<DT, 2>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
    case 3: return launch_prep_ni<DT, 3>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
    case 4: return launch_prep_ni<DT, 4>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
    default: return launch_prep_ni<DT, 5>(ni, mode, x, out, scales, rows, K, waves, mod, stream);
  }
}

}  // namespace

// Pick (iterations per wave, waves per row) so that 1024*NI*W covers K with
// the fewest idle 1024-feature blocks; NI in {3, 4, 1}, W <= 16.  Few rows
// (M <= 2048) take one iteration per wave and more waves per row instead, so
// that enough waves are in flight to cover the load latency.
bool prep_plan(int64_t rows, int64_t K, int* ni_out, int* waves_out) {
  const int64_t blocks = (K + 1023) / 1024;
  {  // tuning override: force the iterations per wave
    const int ni = tuning(kTunePrepNi);
    if (ni == 1 || ni == 3 || ni == 4) {
      const int64_t w = (blocks + ni - 1) / ni;
      if (w <= kMaxWaves) {
        *ni_out = ni;
        *waves_out = (int)w;
        return true;
      }
    }
  }
  if (rows <= 2048 && blocks <= kMaxWaves) {
    *ni_out = 1;
    *waves_out = (int)blocks;
    return true;
  }
  int best_ni = 0, best_w = 0;
  int64_t best_idle = -1;
  const int cand[3] = {3, 4, 1};
  for (int c = 0; c < 3; ++c) {
    const int ni = cand[c];
    const int64_t w = (blocks + ni - 1) / ni;
    if (w > kMaxWaves) continue;
    const int64_t idle = w * ni - blocks;
    if (best_idle < 0 || idle < best_idle) {
      best_idle = idle;
      best_ni = ni;
      best_w = (int)w;
    }
  }
  // Three iterations on more than four waves lose to four iterations on at
  // most four waves with one idle block: at 4608 rows, 15 blocks run 7 % faster
  // as 4 waves x 4 than as 5 waves x 3 (12 blocks stay 4 x 3).
  if (best_ni == 3 && best_w > 4) {
    const int64_t w4 = (blocks + 3) / 4;
    if (w4 <= 4 && w4 * 4 - blocks <= best_idle + 1) {
      best_ni = 4;
      best_w = (int)w4;
      best_idle = w4 * 4 - blocks;
    }
  }
  if (best_idle < 0) return false;
  *ni_out = best_ni;
  *waves_out = best_w;
  return true;
}

namespace {

hipError_t launch_prep_any(const void* x, int dtype, int64_t rows, int64_t K, int log4g, int mode, void* out,
                           float* scales, const Modulation& mod, hipStream_t stream) {
  int ni = 0, waves = 0;
  if (!prep_plan(rows, K, &ni, &waves)) return hipErrorInvalidValue;
  if (rows == 0) return hipSuccess;
  switch (dtype) {
    case kF32: return launch_prep_s<kF32>(log4g, ni, mode, x, out, scales, rows, (int)K, waves, mod, stream);
    case kF16: return launch_prep_s<kF16>(log4g, ni, mode, x, out, scales, rows, (int)K, waves, mod, stream);
    default: return launch_prep_s<kBF16>(log4g, ni, mode, x, out, scales, rows, (int)K, waves, mod, stream);
  }
}

}  // namespace

hipError_t launch_prep(const void* x, int dtype, int64_t rows, int64_t K, int log4g, int mode, void* out,
                       float* scales, hipStream_t stream) {
  Modulation mod{};
  mod.producer = kProPlain;
  return launch_prep_any(x, dtype, rows, K, log4g, mode, out, scales, mod, stream);
}

hipError_t launch_prep_modulated(const void* x, int dtype, int64_t rows, int64_t K, int log4g, int mode,
                                 const void* shift, const void* scale, int64_t rows_per_vector, float eps,
                                 void* out, float* scales, hipStream_t stream) {
  Modulation mod{};
  mod.producer = kProModulate;
  mod.args.shift = shift;
  mod.args.scale = scale;
  mod.args.rows_per_vector = (int)rows_per_vector;
  mod.args.eps = eps;
  return launch_prep_any(x, dtype, rows, K, log4g, mode, out, scales, mod, stream);
}

hipError_t launch_prep_gelu(const void* head, int64_t head_features, int64_t head_stride, const void* x,
                            int64_t x_features, int64_t x_stride, int dtype, int64_t rows, int log4g, int mode,
                            void* out, float* scales, hipStream_t stream) {
  Modulation mod{};
  mod.producer = kProGelu;
  mod.args.head = head;
  mod.args.head_features = (int)head_features;
  mod.args.head_stride = head_stride;
  mod.args.x_stride = x_stride;
  return launch_prep_any(x, dtype, rows, head_features + x_features, log4g, mode, out, scales, mod, stream);
}

}  // namespace convrot
