// qmlp_prep.hip -- activation passes that run before the projection kernels for the many-token
// path: the bfp8 fp16 conversion with per-token scales, and the RMSNorm pass.
#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

// ---------------------------------------------------------------- bfp8 activation prep
//
// x bf16 -> x16 = fp16(x * 2^tx[m]) with a per-token power of two that puts max|x[m]| in
// [2^14, 2^15), and th[m] from the Cauchy-Schwarz bound |h| <= |x_m|^2 max|Wg_n| max|Wu_n| (row
// norms from the packed trailers) so that h * 2^th[m] fits fp16.
//
// One wave per token row, 16-byte loads (H is a multiple of 256, so a row is a whole number of
// 16-byte chunks): the first pass reduces the row's max|x| and sum of squares (lane partials, then
// a fixed xor tree: deterministic), the second converts and writes x16.  Rows of up to
// 64 * kPrepRegCh chunks (H <= 8192) are held in registers between the passes, with every load
// of the row in flight at once; longer rows re-read their chunks (from L2) in the second pass.
constexpr int kPrepRows = 4;    // token rows (waves) per block
constexpr int kPrepRegCh = 16;  // 16-byte chunks per lane held in registers

__global__ __launch_bounds__(64 * kPrepRows) void prep_kernel(const uint16_t* __restrict__ x, int M, int H,
                                                             const Trailer* tg, const Trailer* tu,
                                                             uint16_t* __restrict__ x16, int* __restrict__ tx,
                                                             int* __restrict__ th) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * kPrepRows + (int)(threadIdx.x >> 6);
  if (m >= M) return;  // whole waves
  const u32x4* xr = (const u32x4*)(x + (size_t)m * H);
  const int nch = H / 8;
  const bool in_regs = nch <= 64 * kPrepRegCh;
  float mx = 0.f;
  double ss = 0.0;
  auto reduce = [&](const u32x4& v) {
    float cs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_to_f32((uint16_t)(v[i] & 0xffffu)), hi = bf16_to_f32((uint16_t)(v[i] >> 16));
      mx = fmaxf(mx, fmaxf(fabsf(lo), fabsf(hi)));
      cs = fmaf(lo, lo, cs);
      cs = fmaf(hi, hi, cs);
    }
    ss += (double)cs;
  };
  u32x4 rv[kPrepRegCh];
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kPrepRegCh; ++i)
      if (lane + 64 * i < nch) rv[i] = xr[lane + 64 * i];
#pragma unroll
    for (int i = 0; i < kPrepRegCh; ++i)
      if (lane + 64 * i < nch) reduce(rv[i]);
  } else {
    for (int c = lane; c < nch; c += 64) reduce(xr[c]);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    ss += __shfl_xor(ss, o);
  }
  int e = 0;
  if (mx > 0.f) frexpf(mx, &e);
  const int txm = mx > 0.f ? 15 - e : 0;
  if (lane == 0) {
    const double gn = __longlong_as_double((long long)tg->max_row_norm_bits);
    const double un = __longlong_as_double((long long)tu->max_row_norm_bits);
    const double bound = ss * gn * un * (1.0 + 1.0 / 64.0);
    int eb = 0;
    if (bound > 0.0) frexp(bound, &eb);
    tx[m] = txm;
    th[m] = bound > 0.0 ? 15 - eb : 0;
  }
  u32x4* orow = (u32x4*)(x16 + (size_t)m * H);
  auto convert = [&](const u32x4& v) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_to_f32((uint16_t)(v[i] & 0xffffu)), hi = bf16_to_f32((uint16_t)(v[i] >> 16));
      o[i] = (uint32_t)f32_to_f16_bits(__builtin_amdgcn_ldexpf(lo, txm)) |
             ((uint32_t)f32_to_f16_bits(__builtin_amdgcn_ldexpf(hi, txm)) << 16);
    }
    return o;
  };
  if (in_regs) {
#pragma unroll
    for (int i = 0; i < kPrepRegCh; ++i)
      if (lane + 64 * i < nch) orow[lane + 64 * i] = convert(rv[i]);
  } else {
    for (int c = lane; c < nch; c += 64) orow[c] = convert(xr[c]);
  }
}

// ---------------------------------------------------------------- RMSNorm pass (M > 32)
//
// xn = bf16(x * (1 / sqrt(mean(x^2) + eps)) * (1 + w)): the decoder's ffn_norm
// (docker/qwen-c2-graft/graft/layer.py:110-112,228-237, add_unit_offset) as a separate pass for the
// token counts whose kernels read the activations straight from memory.  One wave per token row,
// 16-byte loads; the row's sum of squares is reduced in a fixed order (deterministic).
__global__ __launch_bounds__(64 * kPrepRows) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                                const uint16_t* __restrict__ w, float eps, int M,
                                                                int H, uint16_t* __restrict__ xn) {
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * kPrepRows + (int)(threadIdx.x >> 6);
  if (m >= M) return;  // whole waves
  const u32x4* xr = (const u32x4*)(x + (size_t)m * H);
  const u32x4* wr = (const u32x4*)w;
  const int nch = H / 8;
  float ss = 0.f;
  for (int c = lane; c < nch; c += 64) {
    const u32x4 v = xr[c];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_to_f32((uint16_t)(v[i] & 0xffffu)), hi = bf16_to_f32((uint16_t)(v[i] >> 16));
      ss = fmaf(lo, lo, ss);
      ss = fmaf(hi, hi, ss);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
  const float rs = 1.0f / sqrtf(ss / (float)H + eps);
  u32x4* orow = (u32x4*)(xn + (size_t)m * H);
  for (int c = lane; c < nch; c += 64) {
    const u32x4 v = xr[c], g = wr[c];
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = bf16_to_f32((uint16_t)(v[i] & 0xffffu)), hi = bf16_to_f32((uint16_t)(v[i] >> 16));
      const float glo = bf16_to_f32((uint16_t)(g[i] & 0xffffu)), ghi = bf16_to_f32((uint16_t)(g[i] >> 16));
      o[i] = (uint32_t)f32_to_bf16(lo * rs * (1.0f + glo)) | ((uint32_t)f32_to_bf16(hi * rs * (1.0f + ghi)) << 16);
    }
    orow[c] = o;
  }
}

int launch_rmsnorm(const void* x, const void* w, float eps, int M, int H, void* xn, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((M + kPrepRows - 1) / kPrepRows), dim3(64 * kPrepRows), 0, s,
                     (const uint16_t*)x, (const uint16_t*)w, eps, M, H, (uint16_t*)xn);
  return check_launch("rmsnorm_kernel");
}

int launch_prep(const ForwardArgs& a, hipStream_t s) {
  const WsLayout L = ws_layout(a.M, a.H, a.I, a.fmt);
  const Trailer* tg = (const Trailer*)(a.wg + trailer_offset(a.I, a.H, a.fmt));
  const Trailer* tu = (const Trailer*)(a.wu + trailer_offset(a.I, a.H, a.fmt));
  hipLaunchKernelGGL(prep_kernel, dim3((a.M + kPrepRows - 1) / kPrepRows), dim3(64 * kPrepRows), 0, s,
                     (const uint16_t*)a.x, a.M, a.H, tg, tu, (uint16_t*)(a.ws + L.x16), (int*)(a.ws + L.tx),
                     (int*)(a.ws + L.th));
  return check_launch("prep_kernel");
}

}  // namespace qmlp
