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

__global__ __launch_bounds__(256) void prep_kernel(const uint16_t* __restrict__ x, int H,
                                                   const Trailer* tg, const Trailer* tu,
                                                   uint16_t* __restrict__ x16, int* __restrict__ tx,
                                                   int* __restrict__ th) {
  __shared__ float smax[256];
  __shared__ double ssum[256];
  __shared__ int sexp;
  const int m = blockIdx.x;
  const uint16_t* xr = x + (size_t)m * H;
  float mx = 0.f;
  double ss = 0.0;
  for (int k = threadIdx.x; k < H; k += 256) {
    const float v = bf16_to_f32(xr[k]);
    mx = fmaxf(mx, fabsf(v));
    ss += (double)v * (double)v;
  }
  smax[threadIdx.x] = mx;
  ssum[threadIdx.x] = ss;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      smax[threadIdx.x] = fmaxf(smax[threadIdx.x], smax[threadIdx.x + s]);
      ssum[threadIdx.x] += ssum[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    int e = 0;
    const float mxa = smax[0];
    if (mxa > 0.f) frexpf(mxa, &e);
    const int txm = mxa > 0.f ? 15 - e : 0;
    const double gn = __longlong_as_double((long long)tg->max_row_norm_bits);
    const double un = __longlong_as_double((long long)tu->max_row_norm_bits);
    const double bound = ssum[0] * gn * un * (1.0 + 1.0 / 64.0);
    int eb = 0;
    if (bound > 0.0) frexp(bound, &eb);
    tx[m] = txm;
    th[m] = bound > 0.0 ? 15 - eb : 0;
    sexp = txm;
  }
  __syncthreads();
  const int txm = sexp;
  uint16_t* orow = x16 + (size_t)m * H;
  for (int k = threadIdx.x; k < H; k += 256)
    orow[k] = f32_to_f16_bits(__builtin_amdgcn_ldexpf(bf16_to_f32(xr[k]), txm));
}

// ---------------------------------------------------------------- RMSNorm pass (M > 16)
//
// xn = bf16(x * (1 / sqrt(mean(x^2) + eps)) * (1 + w)), one block per token row: the decoder's
// ffn_norm (docker/qwen-c2-graft/graft/layer.py:110-112,228-237, add_unit_offset) as a separate
// pass for the token counts whose kernels read the activations straight from memory.  The
// row's sum of squares is reduced in a fixed order (deterministic).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
                                                      float eps, int H, uint16_t* __restrict__ xn) {
  __shared__ float red[256];
  const int m = blockIdx.x;
  const uint16_t* xr = x + (size_t)m * H;
  float ss = 0.f;
  for (int k = threadIdx.x; k < H; k += 256) {
    const float v = bf16_to_f32(xr[k]);
    ss = fmaf(v, v, ss);
  }
  red[threadIdx.x] = ss;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  const float rs = 1.0f / sqrtf(red[0] / (float)H + eps);
  uint16_t* orow = xn + (size_t)m * H;
  for (int k = threadIdx.x; k < H; k += 256) orow[k] = f32_to_bf16(bf16_to_f32(xr[k]) * rs * (1.0f + bf16_to_f32(w[k])));
}

int launch_rmsnorm(const void* x, const void* w, float eps, int M, int H, void* xn, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(256), 0, s, (const uint16_t*)x, (const uint16_t*)w, eps, H,
                     (uint16_t*)xn);
  return check_launch("rmsnorm_kernel");
}

int launch_prep(const ForwardArgs& a, hipStream_t s) {
  const WsLayout L = ws_layout(a.M, a.H, a.I, a.fmt);
  const Trailer* tg = (const Trailer*)(a.wg + trailer_offset(a.I, a.H, a.fmt));
  const Trailer* tu = (const Trailer*)(a.wu + trailer_offset(a.I, a.H, a.fmt));
  hipLaunchKernelGGL(prep_kernel, dim3(a.M), dim3(256), 0, s, (const uint16_t*)a.x, a.H, tg, tu,
                     (uint16_t*)(a.ws + L.x16), (int*)(a.ws + L.tx), (int*)(a.ws + L.th));
  return check_launch("prep_kernel");
}

}  // namespace qmlp
