// Device-side helpers shared by the gfx950 ConvRot kernels.
//
// Rounding model: the reference evaluates every elementwise op of a bf16/f16
// array in float32 and rounds the result back to the array dtype with
// round-to-nearest-even (MLX eager semantics, restated in
// /root/reference/src/convrot_mlx/core.py:84-94,154-157).  `rnd<DT>` is that
// rounding, returning the rounded value widened back to float32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace convrot {

enum DType : int { kF32 = 0, kF16 = 1, kBF16 = 2 };

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Round to bf16 (RNE) and widen back, in one v_cvt_pk_bf16_f32: the packed
// result {0, bf16(x)} read as a 32-bit float is exactly float(bf16(x)).
__device__ __forceinline__ float round_bf16(float x) {
  f32x2 v = {0.0f, x};
  bf16x2 b = __builtin_convertvector(v, bf16x2);
  return __builtin_bit_cast(float, b);
}

__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

template <int DT>
__device__ __forceinline__ float rnd(float x) {
  if constexpr (DT == kBF16) return round_bf16(x);
  else if constexpr (DT == kF16) return round_f16(x);
  else return x;
}

// Element storage type helpers.
template <int DT> struct Elem;
template <> struct Elem<kF32> { using T = float; };
template <> struct Elem<kF16> { using T = _Float16; };
template <> struct Elem<kBF16> { using T = __bf16; };

template <int DT>
__device__ __forceinline__ float to_f32(typename Elem<DT>::T v) { return (float)v; }

// bf16 bits in the low / high half of a 32-bit word -> float32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

// Pack two floats (already bf16-representable or to be rounded RNE) into a
// bf16x2 word, `lo` in bits 0-15.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

// Round a float32 result to the output dtype and store it.
template <int DT>
__device__ __forceinline__ void store_out(void* base, int64_t idx, float v) {
  if constexpr (DT == kBF16) ((__bf16*)base)[idx] = (__bf16)v;
  else if constexpr (DT == kF16) ((_Float16*)base)[idx] = (_Float16)v;
  else ((float*)base)[idx] = v;
}

// Store 4 consecutive outputs (16-, 8- or 8-byte aligned as dtype requires).
template <int DT>
__device__ __forceinline__ void store_out4(void* base, int64_t idx, float a, float b, float c, float d) {
  if constexpr (DT == kBF16) {
    uint2 w = {pack_bf16x2(a, b), pack_bf16x2(c, d)};
    *(uint2*)((__bf16*)base + idx) = w;
  } else if constexpr (DT == kF16) {
    uint2 w = {pack_f16x2(a, b), pack_f16x2(c, d)};
    *(uint2*)((_Float16*)base + idx) = w;
  } else {
    *(float4*)((float*)base + idx) = make_float4(a, b, c, d);
  }
}

// Signed nibbles of one 32-bit word of a CDNA4 weight block, expanded to int8
// scaled by 16: byte j of `lo` is 16*k[j], byte j of `hi` is 16*k[j+4], where
// k[j] is the low nibble and k[j+4] the high nibble of byte j.
__device__ __forceinline__ void nibbles_x16(uint32_t w, uint32_t& lo, uint32_t& hi) {
  lo = (w << 4) & 0xf0f0f0f0u;
  hi = w & 0xf0f0f0f0u;
}

// ---- direct-to-LDS loads (the DMA GEMM pipelines)

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

// The same with 4 bytes per lane (buffer_load_dword ... lds): LDS at
// lds_addr + 4 * lane.  Each dword is range-checked on its own, so a ragged
// end reads zeros exactly from the first dword past `bytes`.
__device__ __forceinline__ void dma4(i32x4_sgpr rsrc, uint32_t voffset, uint32_t lds_addr) {
  asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voffset), "s"(rsrc), "{m0}"(lds_addr) : "memory");
}

// s_waitcnt on vmcnt only (expcnt and lgkmcnt left at "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  asm volatile("" ::: "memory");
}

}  // namespace convrot
