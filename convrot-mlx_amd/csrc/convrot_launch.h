// Host-side launchers of the gfx950 kernels (internal to the library; the
// public ABI is include/convrot_amd.h).  Each returns the launch status; shape
// validation happens in capi.hip before any launcher is called.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/convrot_amd.h"
#include "convrot_device.h"

namespace convrot {

// Overrides of the kernel and plan choice for tuning sweeps and tests, set
// through convrot_set_tuning (capi.hip); -1 means "not set" (automatic choice).
// Nothing reads the environment: production dispatch depends on the shape only.
enum TuneKey : int {
  kTuneGemmTile = 0,     // W4A4 tile: bm | bn << 10 | wm << 20 | wn << 24 | stages << 28 (stages 0: any)
  kTuneGemmSk,           // W4A4 kernel kind: 0 data-parallel, 1 stream-K
  kTuneGemmSkMin,        // shortest stream-K range in k-blocks
  kTuneGemmNoDma,        // 1: the register-staged W4A4 kernel instead of the DMA kernels
  kTuneGemmSmallmMax,    // largest M the few-row W4A4 kernel takes (0: never)
  kTuneW4a4SmallmCfg,    // few-row W4A4 split, as a character code ('A', 'B', 'C', 'F')
  kTuneW4a16Cfg,         // W4A16 kernel, as a character code ('A' .. 'F', 'S', 'T')
  kTuneW4a16Tile,        // W4A16 tiled kernel tile: bm | bn << 10
  kTunePrepNi,           // prep kernel 1024-feature iterations per wave (1, 3 or 4)
  kTuneSkSpinLimit,      // stream-K bounded wait: polls before an owner gives up
  kTuneGemmPersist,      // persistent 4-wave W4A4 kernel: 0 never, G > 0 always, on a grid of G workgroups
  kTuneGemmMfma32,       // 1: the 4-wave 256x256 tile on v_mfma_i32_32x32x32_i8
  kTuneFp6Tile,          // FP6 W4A4 tile: bm | bn << 10
  kTuneCount
};
int tuning(TuneKey key);

// Whether a tile forced through convrot_set_tuning is one the library builds:
// a W4A4 INT8 tile (DMA kernels with ring depth `stages`, 0 for any, or the
// register-staged kernel), an FP6 W4A4 tile, a W4A16 tiled-kernel tile.
bool w4a4_tile_known(int bm, int bn, int wm, int wn, int stages);
bool fp6_tile_known(int bm, int bn);
bool w4a16_tile_known(int bm, int bn);

// The FP6 W4A4 tile the plan (and the fp6_tile override) picks for M x N.
void fp6_plan_tile(int64_t M, int64_t N, int* bm, int* bn);

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

// Device memory of the stream-K W4A4 GEMM: a control block (counters,
// generation, error word, partial-ready flags) and one int32 partial tile per
// workgroup slot.  kSkWorkspaceBytes covers every plan on up to 256 CUs (a
// plan needing more runs data-parallel).  It must be zero-filled before its
// first launch; launches leave it ready for the next one and must not
// overlap in time.
struct Workspace {
  uint8_t* ptr = nullptr;
  size_t bytes = 0;
};
constexpr size_t kSkWorkspaceBytes = 32768 + (size_t)256 * 256 * 256 * 4;

// The stream-K workspace of a W4A4 launch: none (data-parallel plans only; the
// library never allocates one), or a given one (its null pointer: the same).
struct WorkspaceSource {
  enum Kind { kNone, kGiven } kind = kNone;
  Workspace given{};
};

hipError_t launch_w4a4_gemm(const void* act, int act_format, const float* xscales, const uint8_t* qweight,
                            const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K,
                            void* out, int out_dtype, hipStream_t stream,
                            const GatedResidual& gr = GatedResidual{}, WorkspaceSource src = WorkspaceSource{});

// Synchronizes `stream`, then reads and clears the error word of `workspace`
// (nullptr: the no-alloc entry point's static scratch on this device, if set up).  Returns 0
// (no error), 1 (a bounded stream-K wait gave up since the last check; *what
// describes it) or -1 (a HIP call failed).
int w4a4_workspace_status(const void* workspace, hipStream_t stream, const char** what);

// Bytes of stream-K workspace the automatic W4A4 plan of this shape uses when
// kSkWorkspaceBytes are available (0: a data-parallel plan, the few-row kernel
// or the packed-activation kernel), under the current tuning overrides.
size_t w4a4_plan_workspace_bytes(int act_format, int64_t M, int64_t N, int64_t K);

// Static scratch of convrot_w4a4_gemm_noalloc (a file-scope device array, one
// per GPU; no allocation): its size, and its device address on the current
// device.  The first call on a device looks the address up and zero-fills the
// control block with a kernel on `stream`.
constexpr size_t kNoAllocScratchBytes = kSkWorkspaceBytes;
hipError_t noalloc_scratch(hipStream_t stream, Workspace* out);

// w6: FP6 operand blocks (1536 bytes a 16 x 128 block), or with compact_weights
// the compact layout of weights whose codes lie in [-7, 7] (1024 bytes a block).
hipError_t launch_w4a4_gemm_fp6(const uint8_t* act6, const float* xscales, const uint8_t* w6, const float* wscales,
                                const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                                hipStream_t stream, const GatedResidual& gr, bool compact_weights = false);

// Few-row W4A4 kernel (int8 activation codes only); launch_w4a4_gemm routes
// small M here.
hipError_t launch_w4a4_smallm(const int8_t* act, const float* xscales, const uint8_t* qweight,
                              const float* wscales, const float* bias, int64_t M, int64_t N, int64_t K, void* out,
                              int out_dtype, hipStream_t stream, const GatedResidual& gr = GatedResidual{});

// Compute units of the current device (cached per device).
int device_cus();

// The W4A16 weight-streaming kernel can split K over workgroups when the
// caller gives a stream-K workspace (few weight tiles, long K, M <= 32): each
// workgroup stores its float32 partial, and the last of a tile group to
// arrive adds the group's partials in split order (deterministic) and runs
// the epilogue.  In the workspace: one arrival counter per (weight-tile group,
// token tile) on its own 128-byte line in the control block's last 12 KiB
// (after the stream-K words and flags, which this split never touches; each
// counter is back at zero when its launch ends), and the partials from
// kW4a16PartialOffset on (the stream-K partial area: W4A4 and W4A16 launches
// on one stream never overlap in time).
constexpr size_t kW4a16CounterOffset = 20480;
constexpr int kW4a16MaxGroups = 96;
constexpr size_t kW4a16PartialOffset = 32768;
static_assert(kW4a16CounterOffset + (size_t)kW4a16MaxGroups * 128 <= kW4a16PartialOffset, "counters");

hipError_t launch_w4a16_gemm(const void* act, int act_dtype, const uint8_t* qweight, const float* wscales,
                             const float* bias, int64_t M, int64_t N, int64_t K, void* out, int out_dtype,
                             hipStream_t stream, const GatedResidual& gr = GatedResidual{},
                             const Workspace& work = Workspace{});

hipError_t launch_pack_int4(const int8_t* values, int64_t rows, int64_t packed_cols, uint8_t* out,
                            hipStream_t stream);

hipError_t launch_unpack_int4(const uint8_t* packed, int64_t rows, int64_t packed_cols, int8_t* out,
                              hipStream_t stream);

hipError_t launch_repack(const uint8_t* in, int in_layout, uint8_t* out, int out_layout, int64_t N, int64_t K,
                         hipStream_t stream);

hipError_t launch_weight_fp6(const uint8_t* cdna4, uint8_t* fp6, int64_t N, int64_t K, hipStream_t stream);

// CDNA4 int4 weight -> compact FP6 blocks; *minus8 (device int, may be null) is
// zeroed, then set to 1 if a code is -8 (no compact field: those blocks are void).
hipError_t launch_weight_fp6c(const uint8_t* cdna4, uint8_t* fp6c, int* minus8, int64_t N, int64_t K,
                              hipStream_t stream);

}  // namespace convrot
