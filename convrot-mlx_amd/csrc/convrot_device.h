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

// ---- gated residual epilogue
//
// A diffusion transformer block ends every branch in x + gate * linear(...),
// evaluated by torch as two eager ops, each rounding to the array dtype.  The
// W4A4 GEMM can apply it after the linear's own rounding:
//   out[m][n] = dt(residual[m][n] + dt(gate[m / rows_per_gate][n] * dt(lin)))
// with `gate` null meaning a plain residual add, dt(residual + dt(lin)).
// residual is [M][N] contiguous in the output dtype and may be `out` itself:
// every lane loads the residual elements it stores, before storing them, and
// no other lane touches them.  gate rows are gate_stride elements apart.
struct GatedResidual {
  const void* residual;  // null: no residual (plain linear)
  const void* gate;      // null: no gate
  int64_t gate_stride;
  int rows_per_gate;
};

template <int DT>
__device__ __forceinline__ float load_elem(const void* base, int64_t i) {
  return (float)((const typename Elem<DT>::T*)base)[i];
}

// dt(res + dt(g * dt(lin))), returned unrounded (the store rounds it).
template <int DT>
__device__ __forceinline__ float gated_sum(float lin, float res, float g) {
  return res + rnd<DT>(g * rnd<DT>(lin));
}

// Four consecutive element values at element index i (16-byte aligned for
// float32, 8-byte for 16-bit dtypes).
template <int DT>
__device__ __forceinline__ void load_elem4(const void* base, int64_t i, float (&v)[4]) {
  if constexpr (DT == kF32) {
    const float4 f = *(const float4*)((const float*)base + i);
    v[0] = f.x, v[1] = f.y, v[2] = f.z, v[3] = f.w;
  } else {
    const uint2 w = *(const uint2*)((const uint16_t*)base + i);
    if constexpr (DT == kBF16) {
      v[0] = bf16_lo(w.x), v[1] = bf16_hi(w.x), v[2] = bf16_lo(w.y), v[3] = bf16_hi(w.y);
    } else {
      const _Float16* h = (const _Float16*)&w;
      v[0] = (float)h[0], v[1] = (float)h[1], v[2] = (float)h[2], v[3] = (float)h[3];
    }
  }
}

// Residual and gate operands of 4 outputs (row m, columns n..n+3 < N where
// `vec`, with N a multiple of 4; else those < N).  Loading them apart from
// gate_apply4 lets a caller issue the loads of several output groups before
// their stores: the compiler cannot move a load above a store that may alias it.
struct Gated4 {
  float r[4], g[4];
};

template <int DT>
__device__ __forceinline__ void gate_load4(const GatedResidual& gr, int m, int n, int N, bool vec, Gated4& v) {
  const int64_t idx = (int64_t)m * N + n;
  const int64_t gi = (int64_t)(m / gr.rows_per_gate) * gr.gate_stride + n;
#pragma unroll
  for (int j = 0; j < 4; ++j) v.g[j] = 1.0f;
  if (vec) {
    load_elem4<DT>(gr.residual, idx, v.r);
    if (gr.gate) {
      if ((gr.gate_stride & 3) == 0) {
        load_elem4<DT>(gr.gate, gi, v.g);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) v.g[j] = load_elem<DT>(gr.gate, gi + j);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v.r[j] = n + j < N ? load_elem<DT>(gr.residual, idx + j) : 0.0f;
      if (gr.gate && n + j < N) v.g[j] = load_elem<DT>(gr.gate, gi + j);
    }
  }
}

template <int DT>
__device__ __forceinline__ void gate_apply4(const Gated4& v, float (&o)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = gated_sum<DT>(o[j], v.r[j], v.g[j]);
}

template <int DT>
__device__ __forceinline__ void gate_residual4(const GatedResidual& gr, int m, int n, int N, bool vec,
                                               float (&o)[4]) {
  Gated4 v;
  gate_load4<DT>(gr, m, n, N, vec, v);
  gate_apply4<DT>(v, o);
}

// The same for 8 16-bit outputs (row m, columns n..n+7): raw residual and gate
// bits, and the combination with 8 outputs already rounded and packed in `lin`.
struct Gated8 {
  uint4 r, g;
};

template <int DT>
__device__ __forceinline__ void gate_load8(const GatedResidual& gr, int m, int n, int N, bool vec, Gated8& v) {
  static_assert(DT == kBF16 || DT == kF16, "16-bit outputs only");
  const int64_t idx = (int64_t)m * N + n;
  const int64_t gi = (int64_t)(m / gr.rows_per_gate) * gr.gate_stride + n;
  const uint16_t* res = (const uint16_t*)gr.residual + idx;
  const uint16_t* gp = (const uint16_t*)gr.gate + gi;
  const uint32_t one = DT == kBF16 ? 0x3f80u : 0x3c00u;
  if (vec) {
    v.r = *(const uint4*)res;
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (n + 2 * i < N ? (uint32_t)res[2 * i] : 0u) | (n + 2 * i + 1 < N ? (uint32_t)res[2 * i + 1] << 16 : 0u);
    v.r = make_uint4(w[0], w[1], w[2], w[3]);
  }
  if (!gr.gate) {
    v.g = make_uint4(one * 0x10001u, one * 0x10001u, one * 0x10001u, one * 0x10001u);
  } else if (vec && (gr.gate_stride & 7) == 0) {
    v.g = *(const uint4*)gp;
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (n + 2 * i < N ? (uint32_t)gp[2 * i] : one) | (n + 2 * i + 1 < N ? (uint32_t)gp[2 * i + 1] : one) << 16;
    v.g = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

template <int DT>
__device__ __forceinline__ uint4 gate_apply8(const Gated8& v, uint4 lin) {
  const uint32_t lw[4] = {lin.x, lin.y, lin.z, lin.w};
  const uint32_t rw[4] = {v.r.x, v.r.y, v.r.z, v.r.w};
  const uint32_t gw[4] = {v.g.x, v.g.y, v.g.z, v.g.w};
  uint32_t ow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float lo, hi;
    if constexpr (DT == kBF16) {
      lo = gated_sum<DT>(bf16_lo(lw[i]), bf16_lo(rw[i]), bf16_lo(gw[i]));
      hi = gated_sum<DT>(bf16_hi(lw[i]), bf16_hi(rw[i]), bf16_hi(gw[i]));
      ow[i] = pack_bf16x2(lo, hi);
    } else {
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
      const f16x2 l = __builtin_bit_cast(f16x2, lw[i]), r = __builtin_bit_cast(f16x2, rw[i]),
                  g = __builtin_bit_cast(f16x2, gw[i]);
      lo = gated_sum<DT>((float)l.x, (float)r.x, (float)g.x);
      hi = gated_sum<DT>((float)l.y, (float)r.y, (float)g.y);
      ow[i] = pack_f16x2(lo, hi);
    }
  }
  return make_uint4(ow[0], ow[1], ow[2], ow[3]);
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

// 16 bytes per lane at p + OFF through a device-scope (sc1) load, coherent
// across CUs and XCDs with the sc1 stores that wrote it.  Issued through asm,
// so the compiler neither tracks nor waits for it: the caller waits with
// wait_vmcnt and keeps the uses behind that wait.
template <int OFF>
__device__ __forceinline__ i32x4 load_dev16(const void* p) {
  i32x4 v;
  asm volatile("global_load_dwordx4 %0, %1, off offset:%2 sc1" : "=v"(v) : "v"(p), "i"(OFF) : "memory");
  return v;
}

// s_waitcnt on vmcnt only (expcnt and lgkmcnt left at "no wait").
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xf) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
  asm volatile("" ::: "memory");
}

}  // namespace convrot
