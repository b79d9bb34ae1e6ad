// Host-side launchers of the gfx950 kernels (internal to the library; the
// public ABI is include/convrot_amd.h).  Each returns the launch status; shape
// validation happens in capi.hip before any launcher is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/convrot_amd.h"
#include "convrot_device.h"

namespace convrot {

bool prep_plan(int64_t rows, int64_t K, int* ni_out, int* waves_out);

hipError_t launch_prep(const void* x, int dtype, int64_t rows, int64_t K, int log4g, int mode, void* out,
                       float* scales, hipStream_t stream);

// The fused modulated producer (LayerNorm + adaLN modulation, then the
// preparation of launch_prep).
hipError_t launch_prep_modulated(const void* x, int dtype, int64_t rows, int64_t K, int log4g, int mode,
                                 const void* shift, const void* scale, int64_t rows_per_vector, float eps,
                                 void* out, float* scales, hipStream_t stream);

// Preparation of the rows [head | gelu_tanh(x)] (head may have 0 features).
hipError_t launch_prep_gelu(const void* head, int64_t head_features, int64_t head_stride, const void* x,
                            int64_t x_features, int64_t x_stride, int dtype, int64_t rows, int log4g, int mode,
                            void* out, float* scales, hipStream_t stream);

hipError_t launch_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                            const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, hipStream_t stream,
                            const GatedResidual& gr = GatedResidual{});

// Few-row W4A4 kernel (int8 activation codes only); launch_w4a4_gemm routes
// small M here.
hipError_t launch_w4a4_smallm(const int8_t* act, const float* xscales, const uint8_t* qweight,
                              const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K, void* out,
                              int out_dtype, hipStream_t stream, const GatedResidual& gr = GatedResidual{});

// Compute units of the current device (cached per device).
int device_cus();

hipError_t launch_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                             const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                             hipStream_t stream, const GatedResidual& gr = GatedResidual{});

hipError_t launch_pack_int4(const int8_t* values, int64_t rows, int64_t packed_cols, uint8_t* out,
                            hipStream_t stream);

hipError_t launch_unpack_int4(const uint8_t* packed, int64_t rows, int64_t packed_cols, int8_t* out,
                              hipStream_t stream);

hipError_t launch_repack(const uint8_t* in, int in_layout, uint8_t* out, int out_layout, int64_t N, int64_t K,
                         hipStream_t stream);

}  // namespace convrot
