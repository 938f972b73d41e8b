// qmlp_internal.h -- host-side declarations shared by the library's translation units.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace qmlp {

// Error reporting (thread-local message, set by the C ABI layer and the launchers).
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);

// Optional per-kernel timing of the forward pass (qmlp_set_profile_events): slot 0 is the
// gate/up kernel, slot 1 the down kernel.  profile_events() hands out the slot's start / stop
// events while timing is on.
void set_profile_events(const hipEvent_t* ev);
bool profile_events(int slot, hipEvent_t* start, hipEvent_t* stop);

// Launches a hot-path kernel.  While timing is on, the launch goes through hipExtLaunchKernel so
// that the dispatch's own start and end timestamps land in the slot's events (no marker packets
// between the kernels, so the timed kernels run exactly as they do untimed).
// A projection launched in several parts records the start event with its first part and the stop
// event with its last (marks: bit 0 start, bit 1 stop).
template <typename... Args>
void launch_timed_part(int slot, int marks, void (*kern)(Args...), dim3 grid, dim3 block, size_t lds, hipStream_t s,
                       Args... args) {
  hipEvent_t start, stop;
  if (profile_events(slot, &start, &stop))
    hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)lds, s, (marks & 1) ? start : nullptr,
                          (marks & 2) ? stop : nullptr, 0u, args...);
  else
    hipLaunchKernelGGL(kern, grid, block, lds, s, args...);
}
template <typename... Args>
void launch_timed(int slot, void (*kern)(Args...), dim3 grid, dim3 block, size_t lds, hipStream_t s, Args... args) {
  launch_timed_part(slot, 3, kern, grid, block, lds, s, args...);
}

// Load-time kernels (qmlp_pack.hip).
int launch_quantize(const void* w, int rows, int cols, void* q, void* e8, uint32_t* bad, int mbits, hipStream_t s);
int launch_pack(const void* src0, const void* src1, int rows, int cols, int fmt, void* packed, hipStream_t s);
int launch_unpack(const void* packed, int rows, int cols, int fmt, void* q, void* e8, hipStream_t s);
int launch_dequant(const void* packed, int rows, int cols, int fmt, float* out, hipStream_t s);
int launch_fill_zero(void* p, size_t bytes, hipStream_t s);

constexpr int kMaxWorkgroups = 512;  // upper bound used to size the workspace
constexpr int kMaxDim = 1 << 20;      // largest H, I, rows or cols the library accepts

// 2-D split of one projection for the M <= 32 weight-streaming kernel (qmlp_gemv.hip).
struct GemvPlan {
  int G;       // tiles per group
  int S;       // K splits
  int KQ;      // superblocks of the longest K split (splits differ by at most one)
  int Ng;      // tile groups
  int P;       // workgroups = Ng * S
  int maxseg;  // tiles one wave may touch
};
constexpr int kMaxSplit = 16;
// mg: groups of 16 tokens (1 for M <= 16, 2 for M <= 32).
int plan_gemv(int rows, int K, int nmat, int mg, int num_cus, GemvPlan* out);
int gemv_groups(int M);
bool gemv_supported(int M, int H, int I, int num_cus);
// Largest partial-slot buffer any device could need for this projection (workspace size).
size_t gemv_part_bytes(int rows, int K, int nmat, int mg);

// Workspace layout for one forward call.
struct WsLayout {
  size_t counters_gu, counters_d;  // int32 per tile
  size_t tx, th;                   // int32 per token
  size_t x16;                      // f16 [M, H] (bfp8 only)
  size_t h;                        // 16-bit [M, I]
  size_t part_gu, part_d;          // fp32 partial-sum slots
  size_t pss;                      // per-workgroup token sums of squares
  size_t xn;                       // bf16 [M, H] normalised activations (RMSNorm pass)
  size_t split, split_bytes;       // partial tiles of the many-token 32x32 kernels' K splits
  size_t total;
};
WsLayout ws_layout(int M, int H, int I, int fmt);

// Format of down_proj for a forward in `fmt`: the bf4 layout pairs bf4 gate/up with bfp8 down.
inline int down_format(int fmt) { return fmt == 2 ? 1 : fmt; }

// Hot-path launchers.
struct ForwardArgs {
  const void* x;
  const uint8_t* wg;
  const uint8_t* wu;
  const uint8_t* wd;
  const void* residual;
  void* out;
  uint8_t* ws;
  int M, H, I, fmt;
  int out_f32, res_f32;  // fp32 output / fp32 residual instead of bf16
  const void* normw;     // RMSNorm prologue: bf16 [H] weight (gain 1 + w), or null
  float eps;
};
// bfp8: x -> x16 = fp16(x * 2^tx[m]) and the h scale th[m], for all M tokens (qmlp_prep.hip).
int launch_prep(const ForwardArgs& a, hipStream_t s);
// xn = bf16(rmsnorm(x) * (1 + w)) for M token rows (qmlp_prep.hip).
int launch_rmsnorm(const void* x, const void* w, float eps, int M, int H, void* xn, hipStream_t s);
int launch_forward_tiled(const ForwardArgs& a, int num_cus, hipStream_t s);
bool tiled_supported(int M, int H, int I);
// Workspace bytes for the partial tiles of the 32x32 many-token kernels' K-split pieces (0 where
// neither projection of the shape splits on kSplitMaxSlots resident blocks).
constexpr int kSplitMaxSlots = 256;
size_t tiled_split_bytes(int M, int H, int I, int fmt);
int launch_forward_gemv(const ForwardArgs& a, int num_cus, hipStream_t s);
// Stream-K weight-streaming kernels for M <= 32 (qmlp_stream.hip).
int plan_stream(int rows, int K, int num_cus, int* P, int* maxseg);
bool stream_supported(int M, int H, int I, int num_cus);
int launch_forward_stream(const ForwardArgs& a, int num_cus, hipStream_t s);

// Argument validation and dispatch shared by every forward entry point (qmlp_abi.hip).  `fn` names
// the entry point in error messages; normw != null selects the RMSNorm prologue.
int forward_impl(const char* fn, const void* x, const void* wg, const void* wu, const void* wd, const void* residual,
                 void* out, void* ws, size_t ws_bytes, int M, int H, int I, int fmt, int flags, const void* normw,
                 float eps, hipStream_t stream);

}  // namespace qmlp
