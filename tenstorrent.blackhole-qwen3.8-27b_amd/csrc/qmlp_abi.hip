// qmlp_abi.hip -- the extern "C" boundary of libqwen_mlp.so (declared in include/qwen_mlp.h):
// argument validation, error reporting, workspace layout and dispatch.  No call allocates.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>

#include "../../include/qwen_mlp.h"
#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(QMLP_E_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return 0;
}

static thread_local hipEvent_t g_prof[4];
static thread_local bool g_prof_on = false;

void set_profile_events(const hipEvent_t* ev) {
  g_prof_on = ev != nullptr;
  if (ev)
    for (int i = 0; i < 4; ++i) g_prof[i] = ev[i];
}

bool profile_events(int slot, hipEvent_t* start, hipEvent_t* stop) {
  if (!g_prof_on || slot < 0 || slot > 1) return false;
  *start = g_prof[2 * slot];
  *stop = g_prof[2 * slot + 1];
  return true;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

WsLayout ws_layout(int M, int H, int I, int fmt) {
  WsLayout L{};
  size_t off = 0;
  // Arrival counters, per tile (stream-K) or per tile group (split kernel): <= tiles.  They must
  // read zero when a kernel starts and every kernel leaves them zero, so they sit at the same
  // place for every shape, sized for the largest one: a workspace shared by calls of different
  // shapes never has another call's data under a counter.
  L.counters_gu = off;
  off = align256(off + (size_t)(kMaxDim / kTileRows) * 4);
  L.counters_d = off;
  off = align256(off + (size_t)(kMaxDim / kTileRows) * 4);
  static_assert(2 * (kMaxDim / kTileRows) * 4 == QMLP_WS_COUNTER_BYTES, "counter region of the header");
  L.tx = off;
  off = align256(off + (size_t)M * 4);
  L.th = off;
  off = align256(off + (size_t)M * 4);
  L.h = off;
  off = align256(off + (size_t)M * I * 2);
  // partial-sum slots: the stream-K kernel (M <= 32) needs 2 per workgroup of NMAT x 2 token
  // groups x 64 lanes x 16 B, the split kernel (M <= 32) one per (workgroup, tile) of NMAT x MG KB.
  // Sized for every token count up to M (not just M itself), so that a workspace sized for M
  // serves every smaller call: a 16-token call's split needs more slots than a 48-token call's
  // tiled kernels, and the size must never shrink as M grows.
  const size_t sk_gu = (size_t)2 * kMaxWorkgroups * (2 * 2 * 64 * 16);
  const size_t sk_d = (size_t)2 * kMaxWorkgroups * (1 * 2 * 64 * 16);
  size_t gv_gu = 0, gv_d = 0;
  for (int mg = 1; mg <= gemv_groups(std::min(M, 32)); ++mg) {
    gv_gu = std::max(gv_gu, gemv_part_bytes(I, H, 2, mg));
    gv_d = std::max(gv_d, gemv_part_bytes(H, I, 1, mg));
  }
  L.part_gu = off;
  off = align256(off + std::max(sk_gu, gv_gu));
  L.part_d = off;
  off = align256(off + std::max(sk_d, gv_d));
  L.pss = off;
  off = align256(off + (size_t)kMaxWorkgroups * 64 * 4);
  // x16 and xn are read only by the gate/up projection; the many-token down projection reuses
  // both (adjacent) for the partial tiles of its K-split tail.
  L.x16 = off;
  off = align256(off + (fmt != QMLP_FMT_BF16 ? (size_t)M * H * 2 : 0));
  L.xn = off;  // bf16 [M, H]: the normalised activations when the RMSNorm runs as its own pass
  // The partial tiles of the many-token kernels' K-split pieces share xn's place: xn is read only
  // before the gate/up projection (by the activation prep, or by gate/up itself for bf16 weights).
  L.split = off;
  L.split_bytes = tiled_split_bytes(M, H, I, fmt);
  off = align256(off + std::max((size_t)M * H * 2, L.split_bytes));
  L.total = off;
  return L;
}

struct DeviceInfo {
  int ok;  // 1 = gfx950, -1 = unusable
  int num_cus;
};

static DeviceInfo device_info(int dev) {
  static std::mutex mu;
  static DeviceInfo cache[64] = {};
  if (dev < 0 || dev >= 64) return DeviceInfo{-1, 0};
  std::lock_guard<std::mutex> g(mu);
  if (cache[dev].ok == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      cache[dev] = DeviceInfo{-1, 0};
    } else {
      const bool gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
      cache[dev] = DeviceInfo{gfx950 ? 1 : -1, prop.multiProcessorCount};
    }
  }
  return cache[dev];
}

static int current_device_info(DeviceInfo* out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(QMLP_E_DEVICE, "no HIP device");
  *out = device_info(dev);
  if (out->ok != 1) return set_error(QMLP_E_DEVICE, "device %d is not a gfx950 (MI355X) GPU", dev);
  return 0;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static bool known_fmt(int fmt) { return fmt == QMLP_FMT_BF16 || fmt == QMLP_FMT_BFP8 || fmt == QMLP_FMT_BF4; }

static bool shape_ok(int rows, int cols) {
  return rows > 0 && cols > 0 && rows % kTileRows == 0 && cols % kSuperK == 0 && rows <= kMaxDim &&
         cols <= kMaxDim;
}

// Shared validation and dispatch of the forward entry points.
int forward_impl(const char* fn, const void* x, const void* wg, const void* wu, const void* wd, const void* residual,
                 void* out, void* ws, size_t ws_bytes, int M, int H, int I, int fmt, int flags, const void* normw,
                 float eps, hipStream_t stream) {
  if (!x || !wg || !wu || !wd || !out || !ws) return set_error(QMLP_E_NULL, "%s: null pointer", fn);
  if (!known_fmt(fmt)) return set_error(QMLP_E_FORMAT, "%s: unknown format %d", fn, fmt);
  if (flags & ~(QMLP_OUT_F32 | QMLP_RESIDUAL_F32)) return set_error(QMLP_E_FORMAT, "%s: unknown flags 0x%x", fn, flags);
  if (M < 1 || M > 65536) return set_error(QMLP_E_SHAPE, "%s: M=%d out of range [1, 65536]", fn, M);
  if (!shape_ok(16, H) || !shape_ok(16, I))
    return set_error(QMLP_E_SHAPE, "%s: H=%d and I=%d must be positive multiples of 256", fn, H, I);
  // the kernels address one activation matrix ([M, H] or [M, I], up to fp32) with 32-bit offsets
  if ((uint64_t)M * (uint64_t)std::max(H, I) * 4u >= (1ull << 32))
    return set_error(QMLP_E_SHAPE, "%s: M * max(H, I) = %llu exceeds 2^30 elements", fn,
                     (unsigned long long)M * (unsigned long long)std::max(H, I));
  if (!aligned16(x) || !aligned16(wg) || !aligned16(wu) || !aligned16(wd) || !aligned16(out) || !aligned16(ws) ||
      (residual && !aligned16(residual)) || (normw && !aligned16(normw)))
    return set_error(QMLP_E_ALIGN, "%s: every pointer must be 16-byte aligned", fn);
  if (normw && !(eps >= 0.0f)) return set_error(QMLP_E_SHAPE, "%s: eps must be >= 0", fn);
  const size_t xbytes = (size_t)M * H * 2, obytes = (size_t)M * H * ((flags & QMLP_OUT_F32) ? 4 : 2);
  const uintptr_t xb = (uintptr_t)x, ob = (uintptr_t)out;
  if (!(normw && x == out) && xb < ob + obytes && ob < xb + xbytes)
    return set_error(QMLP_E_SHAPE, "%s: out must not overlap x", fn);
  if (residual && residual != out) {
    const size_t rbytes = (size_t)M * H * ((flags & QMLP_RESIDUAL_F32) ? 4 : 2);
    const uintptr_t rb = (uintptr_t)residual;
    if (rb < ob + obytes && ob < rb + rbytes)
      return set_error(QMLP_E_SHAPE, "%s: out may equal residual but must not partially overlap it", fn);
  }
  if (residual == out && residual && ((flags & QMLP_OUT_F32) != 0) != ((flags & QMLP_RESIDUAL_F32) != 0))
    return set_error(QMLP_E_SHAPE, "%s: an in-place residual needs the same dtype as out", fn);
  const WsLayout L = ws_layout(M, H, I, fmt);
  if (ws_bytes < L.total)
    return set_error(QMLP_E_WORKSPACE, "%s: workspace holds %zu bytes, needs %zu", fn, ws_bytes, L.total);
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  ForwardArgs a{x, (const uint8_t*)wg, (const uint8_t*)wu, (const uint8_t*)wd, residual, out, (uint8_t*)ws,
                M, H, I, fmt, (flags & QMLP_OUT_F32) ? 1 : 0, (flags & QMLP_RESIDUAL_F32) ? 1 : 0, normw, eps};
  // M <= 32: split-K weight streaming with LDS-staged activations (the RMSNorm fused into its
  // staging and epilogue); where no such split fits (a K too long for the staged activations, or
  // a device too small for the split's registers), M <= 32: stream-K
  // weight streaming with activations read from L2; larger M: the LDS-tiled matrix-core GEMM.
  // The last two take the RMSNorm as a separate pass.
  if (gemv_supported(M, H, I, di.num_cus)) return launch_forward_gemv(a, di.num_cus, (hipStream_t)stream);
  if (normw) {
    uint8_t* xn = (uint8_t*)ws + L.xn;
    if (int rc = launch_rmsnorm(x, normw, eps, M, H, xn, (hipStream_t)stream)) return rc;
    a.x = xn;
    a.normw = nullptr;
  }
  if (stream_supported(M, H, I, di.num_cus)) return launch_forward_stream(a, di.num_cus, (hipStream_t)stream);
  if (tiled_supported(M, H, I)) return launch_forward_tiled(a, di.num_cus, (hipStream_t)stream);
  return set_error(QMLP_E_SHAPE, "%s: no kernel for M=%d H=%d I=%d", fn, M, H, I);
}

}  // namespace qmlp

using namespace qmlp;

extern "C" {

const char* qmlp_last_error(void) { return g_err; }

// The build stamps the digest of the sources it compiled (see _build.py); a build without one
// reports "unstamped".
#ifndef QMLP_SOURCE_HASH
#define QMLP_SOURCE_HASH "unstamped"
#endif
const char* qmlp_version(void) { return "qwen_mlp 0.3 gfx950 src=" QMLP_SOURCE_HASH; }

size_t qmlp_packed_bytes(int rows, int cols, int fmt) {
  if (!shape_ok(rows, cols) || !known_fmt(fmt)) return 0;
  return packed_total(rows, cols, fmt);
}

static int quantize_impl(const char* fn, const void* w_bf16, int rows, int cols, void* q, void* e8,
                         uint32_t* bad_groups, int mbits, qmlp_stream_t stream) {
  if (!w_bf16 || !q || !e8) return set_error(QMLP_E_NULL, "%s: null pointer", fn);
  if (rows <= 0 || cols <= 0 || cols % 16) return set_error(QMLP_E_SHAPE, "%s: bad shape %dx%d", fn, rows, cols);
  if (!aligned16(w_bf16) || !aligned16(q)) return set_error(QMLP_E_ALIGN, "%s: misaligned pointer", fn);
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  return launch_quantize(w_bf16, rows, cols, q, e8, bad_groups, mbits, (hipStream_t)stream);
}

int qmlp_quantize_bfp8(const void* w_bf16, int rows, int cols, void* q, void* e8, uint32_t* bad_groups,
                       qmlp_stream_t stream) {
  return quantize_impl("qmlp_quantize_bfp8", w_bf16, rows, cols, q, e8, bad_groups, 7, stream);
}

int qmlp_quantize_bf4(const void* w_bf16, int rows, int cols, void* q, void* e8, uint32_t* bad_groups,
                      qmlp_stream_t stream) {
  return quantize_impl("qmlp_quantize_bf4", w_bf16, rows, cols, q, e8, bad_groups, 3, stream);
}

int qmlp_pack(const void* src0, const void* src1, int rows, int cols, int fmt, void* packed, size_t packed_bytes,
              qmlp_stream_t stream) {
  if (!known_fmt(fmt)) return set_error(QMLP_E_FORMAT, "qmlp_pack: unknown format %d", fmt);
  if (!src0 || !packed || (fmt != QMLP_FMT_BF16 && !src1)) return set_error(QMLP_E_NULL, "qmlp_pack: null pointer");
  if (!shape_ok(rows, cols))
    return set_error(QMLP_E_SHAPE, "qmlp_pack: rows must be a multiple of 16 and cols of 256 (%dx%d)", rows, cols);
  if (!aligned16(src0) || !aligned16(packed)) return set_error(QMLP_E_ALIGN, "qmlp_pack: misaligned pointer");
  if (packed_bytes < packed_total(rows, cols, fmt))
    return set_error(QMLP_E_WORKSPACE, "qmlp_pack: packed buffer holds %zu bytes, needs %zu", packed_bytes,
                     packed_total(rows, cols, fmt));
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  return launch_pack(src0, src1, rows, cols, fmt, packed, (hipStream_t)stream);
}

int qmlp_packed_info(const void* packed, int rows, int cols, int fmt, double* max_row_norm, uint32_t* flushed_groups,
                     qmlp_stream_t stream) {
  if (!packed) return set_error(QMLP_E_NULL, "qmlp_packed_info: null pointer");
  if (!shape_ok(rows, cols) || !known_fmt(fmt)) return set_error(QMLP_E_SHAPE, "qmlp_packed_info: bad shape/format");
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  Trailer t;
  const uint8_t* src = (const uint8_t*)packed + trailer_offset(rows, cols, fmt);
  if (hipMemcpyAsync(&t, src, sizeof(t), hipMemcpyDeviceToHost, (hipStream_t)stream) != hipSuccess ||
      hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return set_error(QMLP_E_LAUNCH, "qmlp_packed_info: copy failed");
  if (t.magic != kTrailerMagic) return set_error(QMLP_E_FORMAT, "qmlp_packed_info: buffer was not packed by qmlp_pack");
  double n;
  memcpy(&n, &t.max_row_norm_bits, sizeof(n));
  if (max_row_norm) *max_row_norm = n;
  if (flushed_groups) *flushed_groups = t.flushed_groups;
  return 0;
}

static int unpack_impl(const char* fn, const void* packed, int rows, int cols, int fmt, void* q, void* e8,
                       qmlp_stream_t stream) {
  if (!packed || !q || !e8) return set_error(QMLP_E_NULL, "%s: null pointer", fn);
  if (!shape_ok(rows, cols)) return set_error(QMLP_E_SHAPE, "%s: bad shape %dx%d", fn, rows, cols);
  if (!aligned16(packed) || !aligned16(q)) return set_error(QMLP_E_ALIGN, "%s: misaligned pointer", fn);
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  return launch_unpack(packed, rows, cols, fmt, q, e8, (hipStream_t)stream);
}

int qmlp_unpack_bfp8(const void* packed, int rows, int cols, void* q, void* e8, qmlp_stream_t stream) {
  return unpack_impl("qmlp_unpack_bfp8", packed, rows, cols, QMLP_FMT_BFP8, q, e8, stream);
}

int qmlp_unpack_bf4(const void* packed, int rows, int cols, void* q, void* e8, qmlp_stream_t stream) {
  return unpack_impl("qmlp_unpack_bf4", packed, rows, cols, QMLP_FMT_BF4, q, e8, stream);
}

int qmlp_dequant_packed(const void* packed, int rows, int cols, int fmt, float* out, qmlp_stream_t stream) {
  if (!packed || !out) return set_error(QMLP_E_NULL, "qmlp_dequant_packed: null pointer");
  if (!known_fmt(fmt)) return set_error(QMLP_E_FORMAT, "qmlp_dequant_packed: unknown format");
  if (!shape_ok(rows, cols)) return set_error(QMLP_E_SHAPE, "qmlp_dequant_packed: bad shape %dx%d", rows, cols);
  if (!aligned16(packed) || !aligned16(out)) return set_error(QMLP_E_ALIGN, "qmlp_dequant_packed: misaligned pointer");
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  return launch_dequant(packed, rows, cols, fmt, out, (hipStream_t)stream);
}

size_t qmlp_workspace_bytes(int M, int H, int I, int fmt) {
  if (M < 1 || M > 65536 || !shape_ok(16, H) || !shape_ok(16, I) || !known_fmt(fmt)) return 0;
  return ws_layout(M, H, I, fmt).total;
}

int qmlp_workspace_init(void* ws, size_t ws_bytes, qmlp_stream_t stream) {
  if (!ws) return set_error(QMLP_E_NULL, "qmlp_workspace_init: null pointer");
  if (!aligned16(ws)) return set_error(QMLP_E_ALIGN, "qmlp_workspace_init: misaligned pointer");
  DeviceInfo di;
  if (int rc = current_device_info(&di)) return rc;
  return launch_fill_zero(ws, ws_bytes, (hipStream_t)stream);
}

int qmlp_forward_ex(const void* x, const void* wg, const void* wu, const void* wd, const void* residual, void* out,
                    void* ws, size_t ws_bytes, int M, int H, int I, int fmt, int flags, qmlp_stream_t stream) {
  return forward_impl("qmlp_forward", x, wg, wu, wd, residual, out, ws, ws_bytes, M, H, I, fmt, flags, nullptr, 0.0f,
                      stream);
}

int qmlp_forward_rmsnorm(const void* h, const void* norm_w, float eps, const void* wg, const void* wu, const void* wd,
                         void* out, void* ws, size_t ws_bytes, int M, int H, int I, int fmt, int flags,
                         qmlp_stream_t stream) {
  if (!norm_w) return set_error(QMLP_E_NULL, "qmlp_forward_rmsnorm: null norm weight");
  if (flags & QMLP_RESIDUAL_F32) return set_error(QMLP_E_FORMAT, "qmlp_forward_rmsnorm: the residual is h (bf16)");
  return forward_impl("qmlp_forward_rmsnorm", h, wg, wu, wd, h, out, ws, ws_bytes, M, H, I, fmt, flags, norm_w, eps,
                      stream);
}

int qmlp_forward(const void* x, const void* wg, const void* wu, const void* wd, const void* residual, void* out,
                 void* ws, size_t ws_bytes, int M, int H, int I, int fmt, qmlp_stream_t stream) {
  return qmlp_forward_ex(x, wg, wu, wd, residual, out, ws, ws_bytes, M, H, I, fmt, 0, stream);
}

int qmlp_set_profile_events(void* const* events, int n) {
  if (n == 0) {
    set_profile_events(nullptr);
    return 0;
  }
  if (n != 4 || !events) return set_error(QMLP_E_SHAPE, "qmlp_set_profile_events: need 4 events or 0");
  set_profile_events((hipEvent_t const*)events);
  return 0;
}

int qmlp_plan_split(int rows, int K, int nmat, int M, int num_cus, int* out6) {
  if (!out6) return set_error(QMLP_E_NULL, "qmlp_plan_split: null pointer");
  if (M < 1 || M > 32) return set_error(QMLP_E_SHAPE, "qmlp_plan_split: M=%d out of range [1, 32]", M);
  GemvPlan p;
  if (plan_gemv(rows, K, nmat, gemv_groups(M), num_cus, &p))
    return set_error(QMLP_E_SHAPE, "qmlp_plan_split: no split for %dx%d at M=%d", rows, K, M);
  out6[0] = p.P;
  out6[1] = p.G;
  out6[2] = p.S;
  out6[3] = p.KQ;
  out6[4] = p.Ng;
  out6[5] = p.maxseg;
  return 0;
}

int qmlp_plan_stream(int rows, int K, int num_cus, int* out2) {
  if (!out2) return set_error(QMLP_E_NULL, "qmlp_plan_stream: null pointer");
  int P, maxseg;
  if (plan_stream(rows, K, num_cus, &P, &maxseg)) return set_error(QMLP_E_SHAPE, "qmlp_plan_stream: bad shape %dx%d", rows, K);
  out2[0] = P;
  out2[1] = maxseg;
  return 0;
}

}  // extern "C"
