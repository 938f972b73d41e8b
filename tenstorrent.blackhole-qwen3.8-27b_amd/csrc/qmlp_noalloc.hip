// qmlp_noalloc.hip -- qmlp_forward_noalloc: the forward pass for callers that cannot allocate
// (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// The workspace of qmlp_forward_ex (arrival counters, per-token scales, h, partial-sum slots) lives
// here in a file-scope device array, `scratch`, of kScratchBytes.  Each GPU the library runs on
// holds its own copy until the process ends.  In host code the array's name is only a stand-in for
// the symbol, so the first call on a device (with that device current) looks up that device's
// address with hipGetSymbolAddress and keeps it; every kernel argument and fill uses that address.
//
// Every call on one GPU shares that GPU's array and finds the previous call's contents in it.
// Only the arrival counters must read zero when a forward starts: the array is zero when the code
// object is loaded (a zero-initialised .bss section), and every forward leaves them zero, so no
// call ever clears them.  The first call on a device must come from outside graph capture (the
// address lookup may load the code object on that device); it is refused on a capturing stream.
// Calls that overlap on one GPU (two streams, two host threads) race on the array; callers
// serialise them.
#include <mutex>

#include "../../include/qwen_mlp.h"
#include "qmlp_internal.h"

namespace qmlp {

constexpr size_t kScratchBytes = QMLP_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0 && kScratchBytes >= QMLP_WS_COUNTER_BYTES, "scratch size");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

// This device's address of `scratch`, looked up at the first call on the device (outside graph
// capture).  Thread-safe.
static int scratch_for_current_device(void** out, hipStream_t s) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(QMLP_E_DEVICE, "qmlp_forward_noalloc: no usable HIP device");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess)
      return set_error(QMLP_E_LAUNCH, "qmlp_forward_noalloc: cannot query the stream's capture status");
    if (cs != hipStreamCaptureStatusNone)
      return set_error(QMLP_E_LAUNCH,
                       "qmlp_forward_noalloc: the first call on device %d must be made outside graph capture", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return set_error(QMLP_E_LAUNCH, "qmlp_forward_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s",
                       dev, hipGetErrorString(e));
    addr[dev] = p;
  }
  *out = addr[dev];
  return 0;
}

}  // namespace qmlp

using namespace qmlp;

extern "C" int qmlp_forward_noalloc(const void* x, const void* wg, const void* wu, const void* wd,
                                    const void* residual, void* out, int M, int H, int I, int fmt, int flags,
                                    qmlp_stream_t stream) {
  const size_t need = qmlp_workspace_bytes(M, H, I, fmt);
  if (need == 0) {  // sizes or format out of range
    if (!x || !wg || !wu || !wd || !out) return set_error(QMLP_E_NULL, "qmlp_forward_noalloc: null pointer");
    if (fmt != QMLP_FMT_BF16 && fmt != QMLP_FMT_BFP8 && fmt != QMLP_FMT_BF4)
      return set_error(QMLP_E_FORMAT, "qmlp_forward_noalloc: unknown format %d", fmt);
    return set_error(QMLP_E_SHAPE,
                     "qmlp_forward_noalloc: M=%d H=%d I=%d out of range (1 <= M <= 65536, H and I positive multiples "
                     "of 256)",
                     M, H, I);
  }
  if (need > kScratchBytes)
    return set_error(QMLP_E_WORKSPACE,
                     "qmlp_forward_noalloc: M=%d H=%d I=%d needs %zu bytes of scratch, the library holds %zu "
                     "(use qmlp_forward_ex with a workspace)",
                     M, H, I, need, kScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws, (hipStream_t)stream)) return rc;
  return forward_impl("qmlp_forward_noalloc", x, wg, wu, wd, residual, out, ws, kScratchBytes, M, H, I, fmt, flags,
                      nullptr, 0.0f, (hipStream_t)stream);
}
