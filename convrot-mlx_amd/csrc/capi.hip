// C ABI of the gfx950 ConvRot library (declared in include/convrot_amd.h).
//
// Every entry point validates its arguments before any launch and reports
// failures as a status code plus a thread-local message; messages for the
// conditions the reference checks reuse the reference's wording
// (/root/reference/src/convrot_mlx/core.py:50-61,75-77,431-442,1030-1058).
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>

#include "convrot_launch.h"

namespace convrot {
namespace {
// Tuning overrides, stored as value + 1 so that the zero-initialized table
// means "nothing set".
std::atomic<int> g_tuning[kTuneCount] = {};
}  // namespace

int tuning(TuneKey key) { return g_tuning[key].load(std::memory_order_relaxed) - 1; }
}  // namespace convrot

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return CONVROT_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(CONVROT_ERR_LAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return ok();
}

bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

bool valid_dtype(int dt) { return dt == CONVROT_DTYPE_F32 || dt == CONVROT_DTYPE_F16 || dt == CONVROT_DTYPE_BF16; }

const char* dtype_name(int dt) {
  switch (dt) {
    case CONVROT_DTYPE_F32: return "float32";
    case CONVROT_DTYPE_F16: return "float16";
    case CONVROT_DTYPE_BF16: return "bfloat16";
    default: return "unknown";
  }
}

// core.py:50-61; returns log4(G) or -1
int log4_group(int g) {
  if (g < 4) return -1;
  int s = 0;
  while (g > 1 && g % 4 == 0) {
    g /= 4;
    ++s;
  }
  return g == 1 ? s : -1;
}

constexpr int64_t kMaxFeatures = 65536;
// The GEMM kernels address the packed weights ([ceil(K/128)][ceil(N/16)][1 KB])
// through buffer resources with 32-bit signed offsets: below 2 GiB.
constexpr int64_t kMaxWeightBytes = int64_t(1) << 31;
int64_t packed_weight_bytes(int64_t N, int64_t K) { return ((K + 127) / 128) * ((N + 15) / 16) * 1024; }
// The FP6 GEMM reads each operand through one buffer resource: 32-bit offsets
// (a k-block's offset plus a tile's pieces) must not wrap, so an operand stays
// 1 MiB below 4 GiB.
constexpr int64_t kMaxFp6OperandBytes = (int64_t(1) << 32) - (int64_t(1) << 20);

}  // namespace

extern "C" {

const char* convrot_last_error(void) { return g_err; }

int convrot_set_tuning(const char* name, const char* value) {
  using namespace convrot;
  if (!name) return fail(CONVROT_ERR_INVALID, "null tuning name");
  static const struct {
    const char* name;
    TuneKey key;
  } kNames[] = {{"gemm_tile", kTuneGemmTile},         {"gemm_sk", kTuneGemmSk},
                {"gemm_sk_min", kTuneGemmSkMin},      {"gemm_no_dma", kTuneGemmNoDma},
                {"gemm_smallm_max", kTuneGemmSmallmMax}, {"w4a4_smallm_cfg", kTuneW4a4SmallmCfg},
                {"w4a16_cfg", kTuneW4a16Cfg},         {"w4a16_tile", kTuneW4a16Tile},
                {"prep_ni", kTunePrepNi},             {"sk_spin_limit", kTuneSkSpinLimit},
                {"gemm_persist", kTuneGemmPersist},   {"gemm_mfma32", kTuneGemmMfma32},
                {"fp6_tile", kTuneFp6Tile}};
  int key = -1;
  for (const auto& n : kNames)
    if (strcmp(n.name, name) == 0) key = n.key;
  if (key < 0) return fail(CONVROT_ERR_INVALID, "unknown tuning override '%s'", name);
  int v = -1;
  if (value && value[0]) {
    bool good = true;
    switch (key) {
      case kTuneGemmTile: {
        int bm = 0, bn = 0, wm = 2, wn = 2, st = 0;
        const int got = sscanf(value, "%dx%dw%dx%ds%d", &bm, &bn, &wm, &wn, &st);
        good = got >= 2 && bm > 0 && bm <= 512 && bn > 0 && bn <= 512 && wm > 0 && wm < 16 && wn > 0 && wn < 16 &&
               st >= 0 && st < 8 && w4a4_tile_known(bm, bn, wm, wn, st);
        v = bm | bn << 10 | wm << 20 | wn << 24 | st << 28;
        break;
      }
      case kTuneFp6Tile:
      case kTuneW4a16Tile: {
        int bm = 0, bn = 0;
        char tail = 0;
        good = sscanf(value, "%dx%d%c", &bm, &bn, &tail) == 2 &&
               (key == kTuneFp6Tile ? fp6_tile_known(bm, bn) : w4a16_tile_known(bm, bn));
        v = bm | bn << 10;
        break;
      }
      case kTuneW4a4SmallmCfg:
        good = strchr("ABCF", value[0]) != nullptr && value[1] == '\0';
        v = value[0];
        break;
      case kTuneW4a16Cfg:
        good = strchr("ABCDEFST", value[0]) != nullptr && value[1] == '\0';
        v = value[0];
        break;
      default: {
        char* end = nullptr;
        const long long n = strtoll(value, &end, 10);
        good = end && *end == '\0' && n >= 0 && n <= 0x7fffffff;
        v = (int)n;
      }
    }
    if (!good) return fail(CONVROT_ERR_INVALID, "invalid value '%s' for tuning override '%s'", value, name);
  }
  g_tuning[key].store(v + 1, std::memory_order_relaxed);
  return ok();
}

const char* convrot_version(void) { return "convrot-mi355x 0.1.0 (gfx950)"; }

int64_t convrot_cdna4_bytes(int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  return ((K + 127) / 128) * ((N + 15) / 16) * 1024;
}

int64_t convrot_fp6_bytes(int64_t R, int64_t K) {
  if (R < 0 || K < 0 || K % 128) return -1;
  return (K / 128) * ((R + 15) / 16) * 1536;
}

int convrot_w4a4_fp6_tile(int64_t M, int64_t N, int* bm, int* bn) {
  if (M <= 0 || N <= 0 || !bm || !bn)
    return fail(CONVROT_ERR_INVALID, "FP6 tile query needs M, N > 0 and two result pointers");
  convrot::fp6_plan_tile(M, N, bm, bn);
  return ok();
}

int convrot_prepare(const void* x, int dtype, int64_t rows, int64_t features, int group_size, int mode,
                    void* out, float* scales, void* stream) {
  const bool no_rotate = (mode & CONVROT_PREP_NO_ROTATE) != 0;
  const int kind = mode & ~CONVROT_PREP_NO_ROTATE;
  if (kind != CONVROT_PREP_PACKED && kind != CONVROT_PREP_INT8 && kind != CONVROT_PREP_ROTATE &&
      kind != CONVROT_PREP_FP6)
    return fail(CONVROT_ERR_INVALID, "unknown ConvRot preparation mode %d", mode);
  if (kind == CONVROT_PREP_FP6 && features % 128)
    return fail(CONVROT_ERR_UNSUPPORTED, "FP6 preparation requires features divisible by 128, got %lld",
                (long long)features);
  if (no_rotate && kind == CONVROT_PREP_ROTATE)
    return fail(CONVROT_ERR_INVALID, "rotate mode cannot skip the rotation");
  if (!valid_dtype(dtype)) return fail(CONVROT_ERR_INVALID, "unsupported activation dtype code %d", dtype);
  if (rows < 0 || features <= 0) return fail(CONVROT_ERR_INVALID, "invalid shape (%lld, %lld)", (long long)rows, (long long)features);
  int s = 0;
  if (!no_rotate) {
    s = log4_group(group_size);
    if (s < 0) return fail(CONVROT_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %d", group_size);
    if (s > 5)
      return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot supports groups [4, 16, 64, 256, 1024], got %d", group_size);
    if (features % group_size)
      return fail(CONVROT_ERR_INVALID, "features %lld not divisible by ConvRot group size %d", (long long)features,
                  group_size);
  }
  if (features % 16)
    return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation requires features divisible by 16, got %lld",
                (long long)features);
  if (features > kMaxFeatures)
    return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most %lld features, got %lld",
                (long long)kMaxFeatures, (long long)features);
  if (rows > 0x7fffffff) return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most 2^31-1 rows");
  if (rows == 0) return ok();
  if (!x || !out || (kind != CONVROT_PREP_ROTATE && !scales))
    return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(out, 16)) return fail(CONVROT_ERR_INVALID, "x and out must be 16-byte aligned");
  return launch_status(convrot::launch_prep(x, dtype, rows, features, s, kind, out, scales, (hipStream_t)stream),
                       "convrot_prepare");
}

int convrot_prepare_modulated(const void* x, int dtype, int64_t rows, int64_t features, int group_size, int mode,
                              const void* shift, const void* scale, int64_t rows_per_vector, float eps, void* out,
                              float* scales, void* stream) {
  if (mode & CONVROT_PREP_NO_ROTATE)
    return fail(CONVROT_ERR_INVALID, "the modulated producer always rotates (no CONVROT_PREP_NO_ROTATE)");
  if (mode != CONVROT_PREP_PACKED && mode != CONVROT_PREP_INT8 && mode != CONVROT_PREP_ROTATE &&
      mode != CONVROT_PREP_FP6)
    return fail(CONVROT_ERR_INVALID, "unknown ConvRot preparation mode %d", mode);
  if (!valid_dtype(dtype)) return fail(CONVROT_ERR_INVALID, "unsupported activation dtype code %d", dtype);
  if (rows < 0 || features <= 0) return fail(CONVROT_ERR_INVALID, "invalid shape (%lld, %lld)", (long long)rows, (long long)features);
  if (rows_per_vector <= 0 || rows_per_vector > 0x7fffffff)
    return fail(CONVROT_ERR_INVALID, "rows_per_vector must be in [1, 2^31-1], got %lld", (long long)rows_per_vector);
  if (!(eps >= 0.0f) || eps > 1e30f) return fail(CONVROT_ERR_INVALID, "eps must be finite and non-negative");
  const int s = log4_group(group_size);
  if (s < 0) return fail(CONVROT_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %d", group_size);
  if (s > 5) return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot supports groups [4, 16, 64, 256, 1024], got %d", group_size);
  if (features % group_size)
    return fail(CONVROT_ERR_INVALID, "features %lld not divisible by ConvRot group size %d", (long long)features, group_size);
  if (mode == CONVROT_PREP_FP6 && features % 128)
    return fail(CONVROT_ERR_UNSUPPORTED, "FP6 preparation requires features divisible by 128, got %lld",
                (long long)features);
  if (features % 16)
    return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation requires features divisible by 16, got %lld",
                (long long)features);
  if (features > kMaxFeatures)
    return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most %lld features, got %lld",
                (long long)kMaxFeatures, (long long)features);
  if (rows > 0x7fffffff) return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most 2^31-1 rows");
  if (rows == 0) return ok();
  if (!x || !out || !shift || !scale || (mode != CONVROT_PREP_ROTATE && !scales))
    return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(out, 16) || !aligned(shift, 16) || !aligned(scale, 16))
    return fail(CONVROT_ERR_INVALID, "x, out, shift and scale must be 16-byte aligned");
  return launch_status(convrot::launch_prep_modulated(x, dtype, rows, features, s, mode, shift, scale,
                                                      rows_per_vector, eps, out, scales, (hipStream_t)stream),
                       "convrot_prepare_modulated");
}

int convrot_prepare_gelu(const void* head, int64_t head_features, int64_t head_stride, const void* x,
                         int64_t x_features, int64_t x_stride, int dtype, int64_t rows, int group_size, int mode,
                         void* out, float* scales, void* stream) {
  if (mode & CONVROT_PREP_NO_ROTATE)
    return fail(CONVROT_ERR_INVALID, "the GELU producer always rotates (no CONVROT_PREP_NO_ROTATE)");
  if (mode != CONVROT_PREP_PACKED && mode != CONVROT_PREP_INT8 && mode != CONVROT_PREP_ROTATE &&
      mode != CONVROT_PREP_FP6)
    return fail(CONVROT_ERR_INVALID, "unknown ConvRot preparation mode %d", mode);
  if (!valid_dtype(dtype)) return fail(CONVROT_ERR_INVALID, "unsupported activation dtype code %d", dtype);
  if (rows < 0 || head_features < 0 || x_features <= 0)
    return fail(CONVROT_ERR_INVALID, "invalid GELU producer shape: rows %lld, head %lld, x %lld features",
                (long long)rows, (long long)head_features, (long long)x_features);
  if (head_features % 16 || x_features % 16)
    return fail(CONVROT_ERR_UNSUPPORTED, "the GELU producer requires head and x features divisible by 16, got %lld and %lld",
                (long long)head_features, (long long)x_features);
  const int64_t features = head_features + x_features;
  const int s = log4_group(group_size);
  if (s < 0) return fail(CONVROT_ERR_INVALID, "Regular Hadamard size must be a power of 4, got %d", group_size);
  if (s > 5) return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot supports groups [4, 16, 64, 256, 1024], got %d", group_size);
  if (features % group_size)
    return fail(CONVROT_ERR_INVALID, "features %lld not divisible by ConvRot group size %d", (long long)features, group_size);
  if (mode == CONVROT_PREP_FP6 && features % 128)
    return fail(CONVROT_ERR_UNSUPPORTED, "FP6 preparation requires features divisible by 128, got %lld",
                (long long)features);
  if (features > kMaxFeatures)
    return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most %lld features, got %lld",
                (long long)kMaxFeatures, (long long)features);
  if (x_stride < x_features || (head_features > 0 && head_stride < head_features))
    return fail(CONVROT_ERR_INVALID, "row strides (head %lld, x %lld) shorter than the rows", (long long)head_stride,
                (long long)x_stride);
  if (rows > 0x7fffffff) return fail(CONVROT_ERR_UNSUPPORTED, "fused ConvRot preparation supports at most 2^31-1 rows");
  if (rows == 0) return ok();
  const int64_t esize = dtype == CONVROT_DTYPE_F32 ? 4 : 2;
  if (!x || !out || (head_features > 0 && !head) || (mode != CONVROT_PREP_ROTATE && !scales))
    return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(x, 16) || !aligned(out, 16) || (head_features > 0 && !aligned(head, 16)) || (x_stride * esize) % 16 ||
      (head_features > 0 && (head_stride * esize) % 16))
    return fail(CONVROT_ERR_INVALID, "x, head and out rows must start 16-byte aligned");
  return launch_status(convrot::launch_prep_gelu(head, head_features, head_stride, x, x_features, x_stride, dtype,
                                                 rows, s, mode, out, scales, (hipStream_t)stream),
                       "convrot_prepare_gelu");
}

namespace {

// Argument checks shared by the W4A4 GEMM entry points; CONVROT_OK when the
// launch may proceed (M == 0 or N == 0 included).
int check_w4a4(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
               const float* wscales, int64_t M, int64_t N, int64_t K, void* out, int out_dtype) {
  if (act_format != CONVROT_ACT_PACKED && act_format != CONVROT_ACT_INT8)
    return fail(CONVROT_ERR_INVALID, "unknown activation format %d", act_format);
  if (!valid_dtype(out_dtype)) return fail(CONVROT_ERR_INVALID, "unsupported output dtype code %d", out_dtype);
  if (M < 0 || N < 0 || K <= 0) return fail(CONVROT_ERR_INVALID, "invalid GEMM shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % 32) return fail(CONVROT_ERR_INVALID, "W4A4 GEMM requires K divisible by 32, got %lld", (long long)K);
  if (K > kMaxFeatures)
    return fail(CONVROT_ERR_UNSUPPORTED, "W4A4 GEMM supports K up to %lld, got %lld", (long long)kMaxFeatures, (long long)K);
  if (M > 0x7fffffff || N > 0x7fffffff) return fail(CONVROT_ERR_UNSUPPORTED, "GEMM dimension too large");
  if (packed_weight_bytes(N, K) >= kMaxWeightBytes)
    return fail(CONVROT_ERR_UNSUPPORTED, "W4A4 GEMM packed weights are limited to 2 GiB (N=%lld K=%lld)", (long long)N,
                (long long)K);
  if (M == 0 || N == 0) return ok();
  if (!act || !xscales || !qweight || !wscales || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(act, 16) || !aligned(qweight, 16) || !aligned(out, 16))
    return fail(CONVROT_ERR_INVALID, "act, qweight and out must be 16-byte aligned");
  return ok();
}

}  // namespace

int convrot_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                      const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K, void* out,
                      int out_dtype, void* stream) {
  if (int rc = check_w4a4(act, act_format, xscales, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (M == 0 || N == 0) return ok();
  return launch_status(convrot::launch_w4a4_gemm(act, act_format, xscales, qweight, wscales, bias, M, N, K, out,
                                                 out_dtype, (hipStream_t)stream),
                       "convrot_w4a4_gemm");
}

namespace {

int check_fp6(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales, int64_t M,
              int64_t N, int64_t K, void* out, int out_dtype, int* odt) {
  if (M < 0 || N < 0 || K <= 0 || K % 128 || M > INT32_MAX || N > INT32_MAX || K >= 262144)
    return fail(CONVROT_ERR_INVALID,
                "FP6 W4A4 GEMM: bad shape M=%lld N=%lld K=%lld (K a multiple of 128 below 262144)", (long long)M,
                (long long)N, (long long)K);
  if (convrot_fp6_bytes(M, K) > kMaxFp6OperandBytes || convrot_fp6_bytes(N, K) > kMaxFp6OperandBytes)
    return fail(CONVROT_ERR_UNSUPPORTED,
                "FP6 W4A4 GEMM: an operand of M=%lld or N=%lld rows at K=%lld exceeds %lld FP6 bytes (32-bit "
                "buffer offsets); use the INT8 GEMM",
                (long long)M, (long long)N, (long long)K, (long long)kMaxFp6OperandBytes);
  if (out_dtype != CONVROT_DTYPE_BF16 && out_dtype != CONVROT_DTYPE_F16 && out_dtype != CONVROT_DTYPE_F32)
    return fail(CONVROT_ERR_INVALID, "unsupported output dtype %d", out_dtype);
  *odt = out_dtype == CONVROT_DTYPE_BF16 ? convrot::kBF16 : out_dtype == CONVROT_DTYPE_F16 ? convrot::kF16
                                                                                             : convrot::kF32;
  if (M == 0 || N == 0) return ok();
  if (!act6 || !xscales || !w6 || !wscales || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(act6, 16) || !aligned(w6, 16) || !aligned(out, 16))
    return fail(CONVROT_ERR_INVALID, "act6, w6 and out must be 16-byte aligned");
  return ok();
}

}  // namespace

int convrot_w4a4_gemm_fp6(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                          const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype, void* stream) {
  int odt = 0;
  if (int rc = check_fp6(act6, xscales, w6, wscales, M, N, K, out, out_dtype, &odt)) return rc;
  if (M == 0 || N == 0) return ok();
  return launch_status(convrot::launch_w4a4_gemm_fp6(act6, xscales, w6, wscales, bias, M, N, K, out, odt,
                                                     (hipStream_t)stream, convrot::GatedResidual{}),
                       "convrot_w4a4_gemm_fp6");
}

namespace {

// Checks of the gated-residual arguments shared by both GEMMs (after the GEMM's
// own checks, with M, N > 0); fills `gr` on success.
int check_residual(const void* residual, const void* gate, int64_t gate_stride, int64_t rows_per_gate, int64_t M,
                   int64_t N, convrot::GatedResidual* gr) {
  if (!residual) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(residual, 16) || (gate && !aligned(gate, 16)))
    return fail(CONVROT_ERR_INVALID, "residual and gate must be 16-byte aligned");
  // Any rows_per_gate >= M selects gate row 0 for every output row.
  const int64_t rpg = gate ? (rows_per_gate < M ? rows_per_gate : M) : 1;
  if (gate && (M + rpg - 1) / rpg > 1 && gate_stride < N)
    return fail(CONVROT_ERR_INVALID, "gate rows %lld elements apart overlap (N=%lld)", (long long)gate_stride,
                (long long)N);
  *gr = convrot::GatedResidual{residual, gate, gate ? gate_stride : 0, (int)rpg};
  return ok();
}

}  // namespace

int convrot_w4a4_gemm_residual(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                               const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                               const void* residual, const void* gate, int64_t gate_stride,
                               int64_t rows_per_gate, void* out, int out_dtype, void* stream) {
  if (int rc = check_w4a4(act, act_format, xscales, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  return launch_status(convrot::launch_w4a4_gemm(act, act_format, xscales, qweight, wscales, bias, M, N, K, out,
                                                 out_dtype, (hipStream_t)stream, gr),
                       "convrot_w4a4_gemm_residual");
}

int convrot_w4a4_gemm_fp6_residual(const uint8_t* act6, const float* xscales, const uint8_t* w6,
                                   const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                                   const void* residual, const void* gate, int64_t gate_stride,
                                   int64_t rows_per_gate, void* out, int out_dtype, void* stream) {
  int odt = 0;
  if (int rc = check_fp6(act6, xscales, w6, wscales, M, N, K, out, out_dtype, &odt)) return rc;
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  return launch_status(convrot::launch_w4a4_gemm_fp6(act6, xscales, w6, wscales, bias, M, N, K, out, odt,
                                                     (hipStream_t)stream, gr),
                       "convrot_w4a4_gemm_fp6_residual");
}

int convrot_w4a4_gemm_fp6_compact(const uint8_t* act6, const float* xscales, const uint8_t* w6c,
                                  const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                                  const void* residual, const void* gate, int64_t gate_stride,
                                  int64_t rows_per_gate, void* out, int out_dtype, void* stream) {
  int odt = 0;
  if (int rc = check_fp6(act6, xscales, w6c, wscales, M, N, K, out, out_dtype, &odt)) return rc;
  if (gate && !residual) return fail(CONVROT_ERR_INVALID, "a gate needs a residual");
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (residual)
    if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  return launch_status(convrot::launch_w4a4_gemm_fp6(act6, xscales, w6c, wscales, bias, M, N, K, out, odt,
                                                     (hipStream_t)stream, gr, true),
                       "convrot_w4a4_gemm_fp6_compact");
}

int64_t convrot_w4a4_workspace_bytes(void) { return (int64_t)convrot::kSkWorkspaceBytes; }

int convrot_w4a4_gemm_ws(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                         const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                         const void* residual, const void* gate, int64_t gate_stride, int64_t rows_per_gate,
                         void* workspace, int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  if (int rc = check_w4a4(act, act_format, xscales, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(CONVROT_ERR_INVALID, "invalid workspace (%lld bytes)", (long long)workspace_bytes);
  if (workspace && !aligned(workspace, 256)) return fail(CONVROT_ERR_INVALID, "workspace must be 256-byte aligned");
  if (gate && !residual) return fail(CONVROT_ERR_INVALID, "a gate needs a residual");
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (residual)
    if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  convrot::WorkspaceSource src;
  src.kind = convrot::WorkspaceSource::kGiven;
  src.given = {(uint8_t*)workspace, workspace ? (size_t)workspace_bytes : 0};
  return launch_status(convrot::launch_w4a4_gemm(act, act_format, xscales, qweight, wscales, bias, M, N, K, out,
                                                 out_dtype, (hipStream_t)stream, gr, src),
                       "convrot_w4a4_gemm_ws");
}

int convrot_w4a4_gemm_noalloc(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                              const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                              const void* residual, const void* gate, int64_t gate_stride, int64_t rows_per_gate,
                              void* out, int out_dtype, void* stream) {
  if (int rc = check_w4a4(act, act_format, xscales, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (gate && !residual) return fail(CONVROT_ERR_INVALID, "a gate needs a residual");
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (residual)
    if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  // The plan of convrot_w4a4_gemm_ws with a full workspace; its workspace must fit the static scratch.
  const size_t need = convrot::w4a4_plan_workspace_bytes(act_format, M, N, K);
  if (need > convrot::kNoAllocScratchBytes)
    return fail(CONVROT_ERR_INVALID,
                "convrot_w4a4_gemm_noalloc: the plan for M=%lld N=%lld K=%lld needs %zu bytes of scratch, beyond "
                "the static maximum of %zu",
                (long long)M, (long long)N, (long long)K, need, convrot::kNoAllocScratchBytes);
  convrot::WorkspaceSource src;
  src.kind = convrot::WorkspaceSource::kGiven;
  if (need > 0) {
    if (const hipError_t e = convrot::noalloc_scratch((hipStream_t)stream, &src.given); e != hipSuccess)
      return fail(CONVROT_ERR_LAUNCH, "convrot_w4a4_gemm_noalloc: scratch set-up failed: %s", hipGetErrorString(e));
  }
  return launch_status(convrot::launch_w4a4_gemm(act, act_format, xscales, qweight, wscales, bias, M, N, K, out,
                                                 out_dtype, (hipStream_t)stream, gr, src),
                       "convrot_w4a4_gemm_noalloc");
}

int convrot_w4a4_status(const void* workspace, void* stream) {
  const char* what = nullptr;
  const int rc = convrot::w4a4_workspace_status(workspace, (hipStream_t)stream, &what);
  if (rc < 0) return fail(CONVROT_ERR_LAUNCH, "convrot_w4a4_status: %s", hipGetErrorString(hipGetLastError()));
  if (rc > 0) return fail(CONVROT_ERR_LAUNCH, "%s", what);
  return ok();
}

namespace {

// Argument checks of the W4A16 GEMM entry points; CONVROT_OK when the launch
// may proceed (M == 0 or N == 0 included).
int check_w4a16(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales, int64_t M, int64_t N,
                int64_t K, void* out, int out_dtype) {
  if (act_dtype != CONVROT_DTYPE_F16 && act_dtype != CONVROT_DTYPE_BF16)
    return fail(CONVROT_ERR_INVALID, "MPP W4A16 requires float16 or bfloat16 activation, got %s", dtype_name(act_dtype));
  if (!valid_dtype(out_dtype)) return fail(CONVROT_ERR_INVALID, "unsupported output dtype code %d", out_dtype);
  if (M < 0 || N < 0 || K <= 0) return fail(CONVROT_ERR_INVALID, "invalid GEMM shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  if (K % 32) return fail(CONVROT_ERR_INVALID, "W4A16 GEMM requires K divisible by 32, got %lld", (long long)K);
  if (K > kMaxFeatures)
    return fail(CONVROT_ERR_UNSUPPORTED, "W4A16 GEMM supports K up to %lld, got %lld", (long long)kMaxFeatures, (long long)K);
  if (M > 0x7fffffff || N > 0x7fffffff) return fail(CONVROT_ERR_UNSUPPORTED, "GEMM dimension too large");
  if (packed_weight_bytes(N, K) >= kMaxWeightBytes)
    return fail(CONVROT_ERR_UNSUPPORTED, "W4A16 GEMM packed weights are limited to 2 GiB (N=%lld K=%lld)", (long long)N,
                (long long)K);
  if (M == 0 || N == 0) return ok();
  if (!act || !qweight || !wscales || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(act, 16) || !aligned(qweight, 16) || !aligned(out, 16))
    return fail(CONVROT_ERR_INVALID, "act, qweight and out must be 16-byte aligned");
  return ok();
}

}  // namespace

int convrot_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                       const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype, void* stream) {
  if (int rc = check_w4a16(act, act_dtype, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (M == 0 || N == 0) return ok();
  return launch_status(convrot::launch_w4a16_gemm(act, act_dtype, qweight, wscales, bias, M, N, K, out, out_dtype,
                                                  (hipStream_t)stream),
                       "convrot_w4a16_gemm");
}

int convrot_w4a16_gemm_residual(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                                const float* bias, int64_t M, int64_t N, int64_t K, const void* residual,
                                const void* gate, int64_t gate_stride, int64_t rows_per_gate, void* out,
                                int out_dtype, void* stream) {
  if (int rc = check_w4a16(act, act_dtype, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  return launch_status(convrot::launch_w4a16_gemm(act, act_dtype, qweight, wscales, bias, M, N, K, out, out_dtype,
                                                  (hipStream_t)stream, gr),
                       "convrot_w4a16_gemm_residual");
}

int convrot_w4a16_gemm_ws(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                          const float* bias, int64_t M, int64_t N, int64_t K, const void* residual, const void* gate,
                          int64_t gate_stride, int64_t rows_per_gate, void* workspace, int64_t workspace_bytes,
                          void* out, int out_dtype, void* stream) {
  if (int rc = check_w4a16(act, act_dtype, qweight, wscales, M, N, K, out, out_dtype)) return rc;
  if (workspace_bytes < 0 || (workspace_bytes > 0 && !workspace))
    return fail(CONVROT_ERR_INVALID, "invalid workspace (%lld bytes)", (long long)workspace_bytes);
  if (workspace && !aligned(workspace, 256)) return fail(CONVROT_ERR_INVALID, "workspace must be 256-byte aligned");
  if (gate && !residual) return fail(CONVROT_ERR_INVALID, "a gate needs a residual");
  if (gate && rows_per_gate <= 0)
    return fail(CONVROT_ERR_INVALID, "rows_per_gate must be positive, got %lld", (long long)rows_per_gate);
  if (M == 0 || N == 0) return ok();
  convrot::GatedResidual gr{};
  if (residual)
    if (int rc = check_residual(residual, gate, gate_stride, rows_per_gate, M, N, &gr)) return rc;
  const convrot::Workspace work{(uint8_t*)workspace, workspace ? (size_t)workspace_bytes : 0};
  return launch_status(convrot::launch_w4a16_gemm(act, act_dtype, qweight, wscales, bias, M, N, K, out, out_dtype,
                                                  (hipStream_t)stream, gr, work),
                       "convrot_w4a16_gemm_ws");
}

int convrot_pack_int4(const int8_t* values, int64_t rows, int64_t packed_cols, uint8_t* out, void* stream) {
  if (rows < 0 || packed_cols < 0) return fail(CONVROT_ERR_INVALID, "invalid pack shape");
  if (rows * packed_cols == 0) return ok();
  if (!values || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(values, 2)) return fail(CONVROT_ERR_INVALID, "values must be 2-byte aligned");
  return launch_status(convrot::launch_pack_int4(values, rows, packed_cols, out, (hipStream_t)stream),
                       "convrot_pack_int4");
}

int convrot_unpack_int4(const uint8_t* packed, int64_t rows, int64_t packed_cols, int8_t* out, void* stream) {
  if (rows < 0 || packed_cols < 0) return fail(CONVROT_ERR_INVALID, "invalid unpack shape");
  if (rows * packed_cols == 0) return ok();
  if (!packed || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(out, 2)) return fail(CONVROT_ERR_INVALID, "out must be 2-byte aligned");
  return launch_status(convrot::launch_unpack_int4(packed, rows, packed_cols, out, (hipStream_t)stream),
                       "convrot_unpack_int4");
}

int convrot_repack_weight(const uint8_t* in, int in_layout, uint8_t* out, int out_layout, int64_t N, int64_t K,
                          void* stream) {
  auto valid_layout = [](int l) {
    return l == CONVROT_LAYOUT_NK || l == CONVROT_LAYOUT_KN || l == CONVROT_LAYOUT_CDNA4;
  };
  if (!valid_layout(in_layout) || !valid_layout(out_layout))
    return fail(CONVROT_ERR_INVALID, "unknown weight layout %d -> %d", in_layout, out_layout);
  if (N < 0 || K < 0) return fail(CONVROT_ERR_INVALID, "invalid weight shape (%lld, %lld)", (long long)N, (long long)K);
  if ((in_layout == CONVROT_LAYOUT_KN || out_layout == CONVROT_LAYOUT_KN) && (N % 2))
    return fail(CONVROT_ERR_INVALID, "MPP int4 packing requires even out_features, got %lld", (long long)N);
  if ((in_layout == CONVROT_LAYOUT_NK || out_layout == CONVROT_LAYOUT_NK) && (K % 2))
    return fail(CONVROT_ERR_INVALID, "row-major int4 packing requires even in_features, got %lld", (long long)K);
  if (N == 0 || K == 0) return ok();
  if (!in || !out) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (in == out) return fail(CONVROT_ERR_INVALID, "repack cannot run in place");
  return launch_status(convrot::launch_repack(in, in_layout, out, out_layout, N, K, (hipStream_t)stream),
                       "convrot_repack_weight");
}

int convrot_weight_fp6_compact(const uint8_t* cdna4, uint8_t* fp6c, int* minus8, int64_t N, int64_t K,
                               void* stream) {
  if (N < 0 || K < 0) return fail(CONVROT_ERR_INVALID, "invalid weight shape (%lld, %lld)", (long long)N, (long long)K);
  if (K % 128)
    return fail(CONVROT_ERR_UNSUPPORTED, "FP6 operands require in_features divisible by 128, got %lld",
                (long long)K);
  if ((N == 0 || K == 0) && !minus8) return ok();
  if (((N && K) && (!cdna4 || !fp6c))) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(cdna4, 16) || !aligned(fp6c, 16) || !aligned(minus8, 4))
    return fail(CONVROT_ERR_INVALID, "cdna4 and fp6c must be 16-byte aligned, minus8 4-byte aligned");
  return launch_status(convrot::launch_weight_fp6c(cdna4, fp6c, minus8, N, K, (hipStream_t)stream),
                       "convrot_weight_fp6_compact");
}

int convrot_weight_fp6(const uint8_t* cdna4, uint8_t* fp6, int64_t N, int64_t K, void* stream) {
  if (N < 0 || K < 0) return fail(CONVROT_ERR_INVALID, "invalid weight shape (%lld, %lld)", (long long)N, (long long)K);
  if (K % 128)
    return fail(CONVROT_ERR_UNSUPPORTED, "FP6 operands require in_features divisible by 128, got %lld",
                (long long)K);
  if (N == 0 || K == 0) return ok();
  if (!cdna4 || !fp6) return fail(CONVROT_ERR_INVALID, "null pointer argument");
  if (!aligned(cdna4, 16) || !aligned(fp6, 16)) return fail(CONVROT_ERR_INVALID, "cdna4 and fp6 must be 16-byte aligned");
  return launch_status(convrot::launch_weight_fp6(cdna4, fp6, N, K, (hipStream_t)stream),
                       "convrot_weight_fp6");
}

}  // extern "C"
