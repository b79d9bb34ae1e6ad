/*
 * convrot_amd.h -- C ABI of the MI355X (gfx950) ConvRot W4A4 / W4A16 library.
 *
 * The reference (Lumenbeing/convrot-mlx) has no C FFI: its kernels are Metal
 * source strings dispatched through `mx.fast.metal_kernel` from Python.  Each
 * entry point below replaces one of those kernel launch sites; the citation
 * names the reference function (src/convrot_mlx/core.py:line) whose kernel
 * and argument meaning it takes over.
 *
 * Conventions
 *  - Every pointer is a device pointer the caller allocated; tensors are dense
 *    row-major unless stated.
 *  - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *    Work is enqueued asynchronously; no entry point synchronizes the host
 *    except convrot_w4a4_status.
 *  - Return value: CONVROT_OK or a nonzero status.  convrot_last_error()
 *    returns a thread-local message for the last failure on the calling
 *    thread (the same text the Python layer raises as ValueError).
 *  - Scratch memory.  The library never allocates device memory.  The W4A4
 *    GEMM's stream-K plans (and the W4A16 GEMM's split of K) need a workspace
 *    of convrot_w4a4_workspace_bytes() (a control block plus partial tiles):
 *    convrot_w4a4_gemm_ws and convrot_w4a16_gemm_ws take it from the caller;
 *    convrot_w4a4_gemm and convrot_w4a4_gemm_residual, which have no
 *    workspace, run the data-parallel plans (the same results bit for bit);
 *    convrot_w4a4_gemm_noalloc uses a static device array (one per GPU,
 *    shared by all its calls).  Besides these workspaces and
 *    convrot_set_tuning's overrides the library keeps no global state.
 *    Launches that use one workspace must not overlap in time: keep them on
 *    one stream, and do not replay a captured graph concurrently with other
 *    launches on its capture stream.
 *  - Otherwise calls are reentrant; concurrent calls on different streams are
 *    safe.
 */
#ifndef CONVROT_AMD_H
#define CONVROT_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define CONVROT_DTYPE_F32 0
#define CONVROT_DTYPE_F16 1
#define CONVROT_DTYPE_BF16 2

/* status codes */
#define CONVROT_OK 0
#define CONVROT_ERR_INVALID 1     /* bad shape / dtype / group size / layout */
#define CONVROT_ERR_UNSUPPORTED 2 /* valid request outside this build's kernels */
#define CONVROT_ERR_LAUNCH 3      /* HIP launch or device error */

/* convrot_prepare output modes */
#define CONVROT_PREP_PACKED 0 /* out: uint8 [rows, features/2] packed A4, + scales */
#define CONVROT_PREP_INT8 1   /* out: int8  [rows, features] A4 codes,   + scales */
#define CONVROT_PREP_ROTATE 2 /* out: dtype [rows, features] rotated values (scales unused) */
#define CONVROT_PREP_FP6 3    /* out: FP6 operand blocks of the A4 codes, + scales; features % 128 == 0
                               * (layout: convrot_w4a4_gemm_fp6; convrot_fp6_bytes(rows, features)) */
/* OR-able flag: skip the rotation (quantize_signed_int4_rowwise semantics) */
#define CONVROT_PREP_NO_ROTATE 0x10

/* weight layouts accepted by convrot_repack_weight */
#define CONVROT_LAYOUT_NK 0    /* uint8 [N, K/2], low nibble = even feature   (core.py:1252-1253) */
#define CONVROT_LAYOUT_KN 1    /* uint8 [K, N/2], low nibble = even output    (core.py:1249-1250) */
#define CONVROT_LAYOUT_CDNA4 2 /* uint8 [ceil(K/128)][ceil(N/16)][1024] MFMA tile blocks */

/* activation operand formats for convrot_w4a4_gemm */
#define CONVROT_ACT_PACKED 0 /* uint8 [M, K/2] packed A4 (core.py:1061 mpp_w4a4_matmul) */
#define CONVROT_ACT_INT8 1   /* int8  [M, K]              (core.py:1088 mpp_w4a4_int8_matmul) */

/*
 * Fused activation preparation: normalized regular-Hadamard rotation of each
 * group of `group_size` features, rowwise absmax, symmetric A4 quantization
 * into [-7, 7] and packing, in one pass over x.
 * Replaces the kernels of
 *   metal_fused_prepare_convrot_activation      core.py:425  (mode PACKED)
 *   metal_fused_prepare_convrot_activation_i8   core.py:456  (mode INT8)
 *   metal_fused_rotate_convrot_activation       core.py:487  (mode ROTATE)
 * and, bit-exactly, the eager graphs regular_hadamard (core.py:64),
 * prepare_convrot_activation (core.py:161), quantize_convrot_weight
 * (core.py:514) and, with CONVROT_PREP_NO_ROTATE, quantize_signed_int4_rowwise
 * (core.py:149).
 * x: dtype [rows, features]; group_size in {4, 16, 64, 256, 1024};
 * features % group_size == 0, features % 16 == 0, features <= 65536.
 * scales: float32 [rows] (ignored for ROTATE).
 */
int convrot_prepare(const void* x, int dtype, int64_t rows, int64_t features,
                    int group_size, int mode, void* out, float* scales, void* stream);

/*
 * Fused modulated producer: convrot_prepare applied to
 *   y = rb(rb(rb(1 + scale[v]) * rb((x - mean) * rstd)) + shift[v]),
 *   v = row / rows_per_vector,
 * i.e. a LayerNorm without affine parameters (mean and variance of the row
 * from float64 sums; rstd = 1 / sqrt(var + eps)) followed by the adaLN
 * modulation `(1 + scale) * ln + shift` of a diffusion transformer, each op
 * rounded to the dtype, computed in the same pass as the rotation and
 * quantization (one read of x instead of four passes).  No counterpart in the
 * reference, which runs these as separate ops before ConvRotLinear
 * (/root/reference/examples/flux1_dev/adapter.py:45-70 swaps only the Linears);
 * its design notes name fusing the activation-preparation passes as the
 * remaining optimization target (docs/design.md:54-64).
 * shift, scale: dtype [ceil(rows / rows_per_vector), features]; other
 * arguments as convrot_prepare (group rotation required: no NO_ROTATE).
 */
int convrot_prepare_modulated(const void* x, int dtype, int64_t rows, int64_t features, int group_size, int mode,
                              const void* shift, const void* scale, int64_t rows_per_vector, float eps, void* out,
                              float* scales, void* stream);

/* Fused GELU producer: the preparation of the rows [head | gelu_tanh(x)],
 * features head_features + x_features, in the modes of convrot_prepare.  It has
 * no counterpart in the reference; it fuses the producer that feeds a DiT's
 * MLP-down Linear, linear2(cat(attn, gelu(mlp))) in the FLUX single blocks,
 * into the preparation (the reference names fusing the preparation passes as
 * its open target, /root/reference/docs/design.md:54-64).
 * gelu_tanh is the tanh GELU, nn.GELU(approximate="tanh"), evaluated as a
 * fixed float32 sequence (x^3, fma, exp by Cody-Waite reduction and a degree-7
 * polynomial, one IEEE division) and rounded once to the dtype.
 * head: [rows] rows of head_features elements, head_stride elements apart (NULL
 * when head_features == 0); x: rows of x_features elements, x_stride apart; both
 * 16-byte aligned per row; both feature counts divisible by 16; out and scales
 * as convrot_prepare for features = head_features + x_features. */
int convrot_prepare_gelu(const void* head, int64_t head_features, int64_t head_stride, const void* x,
                         int64_t x_features, int64_t x_stride, int dtype, int64_t rows, int group_size, int mode,
                         void* out, float* scales, void* stream);

/*
 * W4A4 GEMM with fused epilogue:
 *   out[m, n] = out_dtype(((float(sum_k a[m,k] * w[n,k]) * xscales[m]) * wscales[n]) + bias[n])
 * (left to right, no contraction; integer dot exact in int32).
 * Replaces mpp_w4a4_matmul (core.py:1061, act_format PACKED) and
 * mpp_w4a4_int8_matmul (core.py:1088, act_format INT8) -- the MPP TensorOp
 * (core.py:839-874) plus the separate epilogue kernel (core.py:925-937) --
 * with the numerics of reference_w4a4_matmul (core.py:1155-1171).
 * qweight: CONVROT_LAYOUT_CDNA4 bytes for an (N, K) weight.  bias may be NULL
 * (treated as zeros, like the reference's zero bias vector, core.py:1258).
 * K % 32 == 0, K <= 65536.  Without a workspace argument it runs the
 * data-parallel plans only; convrot_w4a4_gemm_ws adds the stream-K plans
 * (few tiles, long K) with the same outputs.
 */
int convrot_w4a4_gemm(const void* act, int act_format, const float* xscales,
                      const uint8_t* qweight, const float* wscales, const float* bias,
                      int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                      void* stream);

/*
 * convrot_w4a4_gemm followed, inside the same kernel, by a gated residual:
 *   lin = the output convrot_w4a4_gemm would store (rounded to out_dtype)
 *   out[m, n] = out_dtype(residual[m, n] + out_dtype(gate[m / rows_per_gate, n] * lin))
 * each op in float32 and rounded to out_dtype, as torch evaluates
 * `residual + gate * linear(x)` eagerly.  No counterpart in the reference: it
 * fuses the consumer of a DiT block's projection Linears (FLUX's
 * x + gate * proj(...) after every attention and MLP branch) into the GEMM, the
 * consumer side of the fused preparation the reference names as its open
 * target (/root/reference/docs/design.md:54-64).
 * residual: [M, N] contiguous, out_dtype, 16-byte aligned; it may be `out`
 * itself (in place) but must not otherwise overlap it.  gate: NULL for a plain
 * residual add (out = out_dtype(residual + lin)), else out_dtype rows of N
 * elements, gate_stride elements apart, 16-byte aligned, not overlapping out;
 * output row m reads gate row m / rows_per_gate (rows_per_gate >= 1; any value
 * >= M broadcasts gate row 0).  Other arguments as convrot_w4a4_gemm.
 */
int convrot_w4a4_gemm_residual(const void* act, int act_format, const float* xscales,
                               const uint8_t* qweight, const float* wscales, const float* bias,
                               int64_t M, int64_t N, int64_t K, const void* residual,
                               const void* gate, int64_t gate_stride, int64_t rows_per_gate,
                               void* out, int out_dtype, void* stream);

/*
 * Bytes of stream-K workspace the W4A4 GEMM can use (any shape, up to 256
 * CUs).  No counterpart in the reference (MLX allocates kernel outputs,
 * core.py:1106-1113, and its TensorOp needs no scratch).
 */
int64_t convrot_w4a4_workspace_bytes(void);

/*
 * convrot_w4a4_gemm / convrot_w4a4_gemm_residual (residual NULL: the plain
 * GEMM; gate and its arguments as there) with a caller-provided workspace:
 * `workspace` is device memory of `workspace_bytes`, 256-byte aligned,
 * zero-filled before its first use and then reused unchanged by later calls
 * (each call leaves it ready for the next); NULL or fewer bytes than a
 * stream-K plan needs restricts the call to data-parallel plans.  Calls that
 * share a workspace must not overlap in time.  Replaces the same launch sites
 * as convrot_w4a4_gemm (core.py:1061, 1088); the Python layer uses this form
 * with a workspace it allocates through torch.
 */
int convrot_w4a4_gemm_ws(const void* act, int act_format, const float* xscales,
                         const uint8_t* qweight, const float* wscales, const float* bias,
                         int64_t M, int64_t N, int64_t K, const void* residual,
                         const void* gate, int64_t gate_stride, int64_t rows_per_gate,
                         void* workspace, int64_t workspace_bytes, void* out, int out_dtype,
                         void* stream);

/*
 * Reports whether a stream-K owner's bounded wait gave up (a partial tile
 * that never arrived; that owner wrote NaN over its output tile instead of a
 * silently wrong value) since the last call: synchronizes `stream`, reads and
 * clears the error word of `workspace` (NULL: the static scratch of
 * convrot_w4a4_gemm_noalloc on the current GPU, if a call set it up).
 * Returns CONVROT_ERR_LAUNCH with a message if so, else CONVROT_OK.
 * Not callable under graph capture.  No counterpart in the reference (its
 * kernels have no error path, core.py:1106-1120).
 */
int convrot_w4a4_status(const void* workspace, void* stream);

/*
 * convrot_w4a4_gemm_ws without a workspace argument and without any
 * allocation: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference (MLX allocates every kernel output itself,
 * core.py:1106-1113).  It runs the plan convrot_w4a4_gemm_ws runs with a full
 * workspace (stream-K where that is faster; outputs the same bits as
 * convrot_w4a4_gemm), taking the stream-K workspace from a static device array of
 * 64 MiB + 32 KiB per GPU (kept until the process ends), which covers every
 * plan on up to 256 CUs; a plan that would need more is rejected with
 * CONVROT_ERR_INVALID.  The first call on a GPU looks up that array's address
 * and zero-fills its control block with a kernel on `stream`; it calls no
 * hipMalloc or hipFree.  Every call on one GPU shares the array: calls that
 * overlap in time on one GPU (other streams, concurrent graph replays) race,
 * so keep them on one stream.  convrot_w4a4_status(NULL, stream) reports a
 * bounded-wait give-up of these calls too.
 */
int convrot_w4a4_gemm_noalloc(const void* act, int act_format, const float* xscales,
                              const uint8_t* qweight, const float* wscales, const float* bias,
                              int64_t M, int64_t N, int64_t K, const void* residual,
                              const void* gate, int64_t gate_stride, int64_t rows_per_gate,
                              void* out, int out_dtype, void* stream);

/*
 * W4A16 GEMM: out[m, n] = out_dtype((dot_f32(act[m, :], w[n, :]) * wscales[n]) + bias[n]).
 * Replaces mpp_w4a16_matmul (core.py:1123-1152): the MPP float x int4 TensorOp
 * (core.py:877-912) plus the elementwise epilogue (core.py:1151-1152).
 * act: act_dtype in {F16, BF16}, [M, K], already rotated.  qweight: CDNA4 layout.
 */
int convrot_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight,
                       const float* wscales, const float* bias, int64_t M, int64_t N,
                       int64_t K, void* out, int out_dtype, void* stream);

/*
 * convrot_w4a16_gemm followed, in the same kernel, by the gated residual of
 * convrot_w4a4_gemm_residual (same arguments, rounding and aliasing rules):
 *   out[m, n] = out_dtype(residual[m, n] + out_dtype(gate[m / rows_per_gate, n] * lin)).
 * No counterpart in the reference (see convrot_w4a4_gemm_residual).
 */
int convrot_w4a16_gemm_residual(const void* act, int act_dtype, const uint8_t* qweight,
                                const float* wscales, const float* bias, int64_t M, int64_t N,
                                int64_t K, const void* residual, const void* gate,
                                int64_t gate_stride, int64_t rows_per_gate, void* out,
                                int out_dtype, void* stream);

/*
 * convrot_w4a16_gemm / _residual (residual and gate may be NULL) with a
 * caller-provided workspace: the same zero-filled stream-K workspace that
 * convrot_w4a4_gemm_ws takes (convrot_w4a4_workspace_bytes() bytes, 256-byte
 * aligned; both GEMMs may share one per stream, launches on it must not
 * overlap in time).  With it the weight-streaming kernel may split K over
 * workgroups (9 <= M <= 32, N <= 4608, K >= 6144: 12288 -> 3072 runs on every
 * CU and reads each weight byte once); the last workgroup of each tile group adds
 * the float32 partials in a fixed order, so results are deterministic, and
 * leaves the workspace ready for the next launch.  workspace = NULL (0 bytes)
 * gives convrot_w4a16_gemm's plan.  The summation order differs from the
 * unsplit kernel's, within the float32 accumulation bound.
 * Replaces mpp_w4a16_matmul (core.py:1123-1152), as convrot_w4a16_gemm.
 */
int convrot_w4a16_gemm_ws(const void* act, int act_dtype, const uint8_t* qweight,
                          const float* wscales, const float* bias, int64_t M, int64_t N,
                          int64_t K, const void* residual, const void* gate,
                          int64_t gate_stride, int64_t rows_per_gate, void* workspace,
                          int64_t workspace_bytes, void* out, int out_dtype, void* stream);

/* pack_signed_int4 (core.py:97-105): int8 [rows, 2*packed_cols] -> uint8 [rows, packed_cols]. */
int convrot_pack_int4(const int8_t* values, int64_t rows, int64_t packed_cols, uint8_t* out,
                      void* stream);

/* metal_unpack_signed_int4 (core.py:1014-1027, kernel :915-922):
 * uint8 [rows, packed_cols] -> int8 [rows, 2*packed_cols] in [-8, 7]. */
int convrot_unpack_int4(const uint8_t* packed, int64_t rows, int64_t packed_cols, int8_t* out,
                        void* stream);

/*
 * Lossless weight re-layout between CONVROT_LAYOUT_* for an (N, K) weight.
 * NK -> KN is repack_nk_weight_for_mpp (core.py:123-133, needs even N);
 * KN -> NK is repack_mpp_weight_to_nk (core.py:136-146, needs even K);
 * NK/KN <-> CDNA4 is this build's tile layout (zero padding; exact inverse).
 */
int convrot_repack_weight(const uint8_t* in, int in_layout, uint8_t* out, int out_layout,
                          int64_t N, int64_t K, void* stream);

/* Size in bytes of a CDNA4-layout weight for an (N, K) weight. */
int64_t convrot_cdna4_bytes(int64_t N, int64_t K);

/*
 * FP6 operand path.  A code v in [-8, 7] is stored as the FP6 (OCP MX e2m3)
 * encoding of v/8: for |v| <= 7 the subnormal with mantissa |v| (a
 * sign-magnitude field, zero as +0), and -1.0 for -8.  gfx950's FP6 matrix
 * instruction (v_mfma_scale_f32_16x16x128_f8f6f4, both operand scales 2^3)
 * then sums the exact products v*w in float32, exactly for K < 262,144
 * (|sum| <= 64 K < 2^24), at twice the INT8 instruction's rate.  So the same
 * GEMM, with the same outputs bit for bit, runs on operands re-encoded as
 * FP6: no counterpart in the reference, whose TensorOp multiplies the int4
 * codes as int8 (core.py:839-874).
 *
 * Operand layout (activations by row, weights by output column): blocks of 16
 * rows x 128 features, 1536 bytes each, ordered [K/128][ceil(R/16)]; lane
 * L = 16 q + r of a block holds row r's features 32 q + i (i = 0 .. 31) as a
 * 24-byte stream (feature i at bits 6i .. 6i+5, little-endian), stream bytes
 * 0 .. 15 at byte 16 L and 16 .. 23 at byte 1024 + 8 L.  K % 128 == 0.
 */

/* Bytes of the FP6 operand blocks of an (R, K) operand (R rows or columns). */
int64_t convrot_fp6_bytes(int64_t R, int64_t K);

/*
 * The BM x BN tile convrot_w4a4_gemm_fp6 runs for an M x N product (the
 * automatic plan, or the fp6_tile tuning override): an introspection call for
 * sweeps and tests, no counterpart in the reference.
 */
int convrot_w4a4_fp6_tile(int64_t M, int64_t N, int* bm, int* bn);

/*
 * CDNA4-layout weight -> FP6 operand blocks (an offline conversion, like
 * convrot_repack_weight); every int4 code, -8 included, has an FP6 field.
 * K % 128 == 0 (else CONVROT_ERR_UNSUPPORTED).
 */
int convrot_weight_fp6(const uint8_t* cdna4, uint8_t* fp6, int64_t N, int64_t K, void* stream);

/*
 * convrot_w4a4_gemm on FP6 operands: act6 from convrot_prepare(..., CONVROT_PREP_FP6,
 * ...), w6 from convrot_weight_fp6.  Same epilogue and outputs, bit for bit, as
 * convrot_w4a4_gemm with act_format CONVROT_ACT_INT8 (out_dtype f32, f16 or
 * bf16); K a multiple of 128 below 262144.  Each operand is addressed with
 * 32-bit offsets: convrot_fp6_bytes(M, K) and convrot_fp6_bytes(N, K) must be
 * at most 2^32 - 2^20, else CONVROT_ERR_UNSUPPORTED (the INT8 GEMM has no such
 * limit).  Replaces the same launch site (core.py:1088-1120).
 */
int convrot_w4a4_gemm_fp6(const uint8_t* act6, const float* xscales, const uint8_t* w6,
                          const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                          void* out, int out_dtype, void* stream);

/*
 * convrot_w4a4_gemm_fp6 followed by the gated residual of
 * convrot_w4a4_gemm_residual (same arguments and rounding; no counterpart in
 * the reference).
 */
int convrot_w4a4_gemm_fp6_residual(const uint8_t* act6, const float* xscales, const uint8_t* w6,
                                   const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                                   const void* residual, const void* gate, int64_t gate_stride,
                                   int64_t rows_per_gate, void* out, int out_dtype, void* stream);

/*
 * Compact FP6 weights (no counterpart in the reference): a weight whose codes
 * all lie in [-7, 7] -- every weight the reference's quantization produces
 * (core.py:154-158 clips to +-7) -- has FP6 fields whose two exponent bits are
 * zero.  The compact layout drops them: blocks of 16 rows x 128 features,
 * 1024 bytes each (convrot_cdna4_bytes(N, K) in all), ordered [K/128][ceil(N/16)];
 * lane L of a block holds at byte 16 L four dwords I0..I3 built from the
 * lane's six FP6 stream dwords D0..D5 (the operand layout above) as
 *   I0 = (D0 & ~Z0) | (D2 & Z0)   I1 = (D1 & ~Z1) | (D2 & Z1)
 *   I2 = (D3 & ~Z0) | (D5 & Z0)   I3 = (D4 & ~Z1) | (D5 & Z1)
 * with Z0 = 0x18618618 and Z1 = 0x86186186 (the exponent bits of D0 and D1).
 *
 * convrot_weight_fp6_compact converts a CDNA4-layout weight (K % 128 == 0).
 * minus8 (a device int, or NULL) is zeroed, then set to 1 if a code is -8:
 * such a weight has no compact form (use convrot_weight_fp6) and the output
 * blocks are void.
 */
int convrot_weight_fp6_compact(const uint8_t* cdna4, uint8_t* fp6c, int* minus8, int64_t N, int64_t K,
                               void* stream);

/*
 * convrot_w4a4_gemm_fp6 (residual NULL) or convrot_w4a4_gemm_fp6_residual on
 * a compact FP6 weight w6c: the GEMM expands each weight fragment to the
 * operand in registers (four bit operations per 16 codes), reading two thirds
 * of the weight bytes.  Same outputs bit for bit.  Replaces the same launch
 * site (core.py:1088-1120).
 */
int convrot_w4a4_gemm_fp6_compact(const uint8_t* act6, const float* xscales, const uint8_t* w6c,
                                  const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                                  const void* residual, const void* gate, int64_t gate_stride,
                                  int64_t rows_per_gate, void* out, int out_dtype, void* stream);

/* Thread-local message of the last failed call on this thread ("" if none). */
const char* convrot_last_error(void);

/*
 * Tuning override: force one of the library's kernel / plan choices for
 * tuning sweeps and tests (value NULL or "" restores the automatic choice,
 * which depends on the shape only).  Process-wide; the library reads no
 * environment variables.  No counterpart in the reference (its kernel choice
 * is the backend name, core.py:1231-1242).  Names and values:
 *   gemm_tile        "BMxBN[wWMxWN[sS]]"  W4A4 tile (and ring depth S)
 *   gemm_sk          "0" | "1"            W4A4 data-parallel / stream-K kernel
 *   gemm_sk_min      k-blocks             shortest stream-K range
 *   gemm_no_dma      "1"                  register-staged int8 W4A4 kernel
 *   gemm_smallm_max  rows                 largest M of the few-row W4A4 kernel (0: never)
 *   w4a4_smallm_cfg  "A" | "B" | "C" | "F"  few-row W4A4 work split
 *   w4a16_cfg        "A" .. "F" | "S" | "T"  W4A16 split (A .. F), split K over workgroups
 *                                        (S, with a workspace) or tiled kernel
 *   w4a16_tile       "BMxBN"              W4A16 tiled-kernel tile
 *   prep_ni          "1" | "3" | "4"      prep kernel 1024-feature blocks per wave
 *   sk_spin_limit    polls                stream-K bounded wait before giving up
 *   gemm_persist     "0" | workgroups     persistent 4-wave W4A4 kernel: never, or always
 *                                         on a grid of that many workgroups
 *   gemm_mfma32      "0" | "1"            4-wave 256x256 W4A4 tile on 32x32x32 MFMAs: never,
 *                                         or always (plain 16-bit outputs)
 *   fp6_tile         "BMxBN"              FP6 W4A4 tile: 256x256, 256x224, 128x256, 128x192 or 128x128
 * Returns CONVROT_ERR_INVALID for an unknown name, a malformed value or a
 * tile the library does not build.
 */
int convrot_set_tuning(const char* name, const char* value);

/* Library version string. */
const char* convrot_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CONVROT_AMD_H */
