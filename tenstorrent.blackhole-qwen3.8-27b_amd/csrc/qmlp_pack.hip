// qmlp_pack.hip -- load-time weight preparation kernels: canonical bfp8 quantisation, packing into
// the tiled layout (qmlp_common.h), the inverse unpack, and an audit dequantiser that reuses the
// GEMM's in-register dequant routine.
#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

// ---------------------------------------------------------------- canonical quantisation
//
// One thread per 16-value group.  Exact integer arithmetic on the bf16 words: a value is
// sig * 2^ex0 with sig < 256; its frexp exponent is bitlen(sig) + ex0.  The shared exponent is the
// largest of the group; q = round-half-even(sig * 2^(ex0 - (e8-127))) clamped to 2^MB - 1.
// MB magnitude bits: 7 (bfp8) or 3 (bf4).
template <int MB>
__global__ void quantize_kernel(const uint16_t* __restrict__ w, int rows, int cols, int8_t* __restrict__ q,
                                uint8_t* __restrict__ e8, uint32_t* bad) {
  const int groups = cols / 16;
  const long gid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (long)rows * groups) return;
  const int r = (int)(gid / groups), g = (int)(gid % groups);
  const uint16_t* src = w + (size_t)r * cols + (size_t)g * 16;
  const u32x4 lo = *(const u32x4*)src;
  const u32x4 hi = *(const u32x4*)(src + 8);
  uint16_t v[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = (uint16_t)(lo[i] & 0xffffu);
    v[2 * i + 1] = (uint16_t)(lo[i] >> 16);
    v[8 + 2 * i] = (uint16_t)(hi[i] & 0xffffu);
    v[8 + 2 * i + 1] = (uint16_t)(hi[i] >> 16);
  }
  int sig[16], ex0[16];
  int shared = -100000;
  bool finite = true, any = false;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int ef = (v[i] >> 7) & 0xff, mf = v[i] & 0x7f;
    if (ef == 0xff) finite = false;
    if (ef == 0) {
      sig[i] = mf;
      ex0[i] = -133;
    } else {
      sig[i] = 128 | mf;
      ex0[i] = ef - 134;
    }
    if (sig[i]) {
      any = true;
      const int e = (32 - __clz(sig[i])) + ex0[i];
      shared = e > shared ? e : shared;
    }
  }
  uint32_t out[4] = {0u, 0u, 0u, 0u};
  uint8_t ebyte = 0;
  if (!finite) {
    if (bad) atomicAdd(bad, 1u);
  } else if (any) {
    int e = shared + 127 - MB;
    e = e < 1 ? 1 : (e > 254 ? 254 : e);
    ebyte = (uint8_t)e;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int s = (e - 127) - ex0[i];  // right shift, >= 1 by construction
      int m;
      if (s >= 10) {
        m = 0;  // sig < 2^8, so sig / 2^s < 1/2
      } else {
        m = sig[i] >> s;
        const int rem = sig[i] & ((1 << s) - 1), half = 1 << (s - 1);
        if (rem > half || (rem == half && (m & 1))) ++m;
      }
      m = m > (1 << MB) - 1 ? (1 << MB) - 1 : m;
      const int qv = (v[i] & 0x8000) ? -m : m;
      out[i / 4] |= ((uint32_t)(qv & 0xff)) << (8 * (i % 4));
    }
  }
  *(u32x4*)(q + (size_t)r * cols + (size_t)g * 16) = u32x4{out[0], out[1], out[2], out[3]};
  e8[(size_t)r * groups + g] = ebyte;
}

// ---------------------------------------------------------------- packing

// Writes the whole 256-byte trailer (zero padding), so a packed buffer's bytes depend only on the
// weights -- packed buffers compare bit-for-bit and cache files are reproducible.
__global__ void trailer_init_kernel(Trailer* t) {
  uint32_t* words = (uint32_t*)t;
  for (int i = threadIdx.x; i < kTrailer / 4; i += blockDim.x) words[i] = 0u;
  __syncthreads();
  if (threadIdx.x == 0) t->magic = kTrailerMagic;
}

// One workgroup (256 threads) per row: row base exponent, rowexp, L2 norm, flushed-group count.
__global__ void rowinfo_bfp8_kernel(const int8_t* __restrict__ q, const uint8_t* __restrict__ e8,
                                    int rows, int cols, int* __restrict__ rowexp, Trailer* trailer) {
  __shared__ int smax[256];
  __shared__ double ssum[256];
  __shared__ unsigned sflush[256];
  const int r = blockIdx.x, groups = cols / 16;
  const uint8_t* er = e8 + (size_t)r * groups;
  int mx = 0;
  for (int g = threadIdx.x; g < groups; g += 256) mx = max(mx, (int)er[g]);
  smax[threadIdx.x] = mx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) smax[threadIdx.x] = max(smax[threadIdx.x], smax[threadIdx.x + s]);
    __syncthreads();
  }
  const int base = smax[0];
  double acc = 0.0;
  unsigned flushed = 0;
  for (int g = threadIdx.x; g < groups; g += 256) {
    const int e = er[g];
    if (!e) continue;
    if (e - base + 20 < 1) ++flushed;
    const int8_t* qg = q + (size_t)r * cols + (size_t)g * 16;
    int sq = 0;
    for (int i = 0; i < 16; ++i) sq += (int)qg[i] * (int)qg[i];
    acc += ldexp((double)sq, 2 * (e - 127));
  }
  ssum[threadIdx.x] = acc;
  sflush[threadIdx.x] = flushed;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      ssum[threadIdx.x] += ssum[threadIdx.x + s];
      sflush[threadIdx.x] += sflush[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    rowexp[r] = base - 132;
    const double n = sqrt(ssum[0]);
    atomicMax(&trailer->max_row_norm_bits, (unsigned long long)__double_as_longlong(n));
    if (sflush[0]) atomicAdd(&trailer->flushed_groups, sflush[0]);
  }
}

__global__ void rowinfo_bf16_kernel(const uint16_t* __restrict__ w, int rows, int cols,
                                    int* __restrict__ rowexp, Trailer* trailer) {
  __shared__ double ssum[256];
  const int r = blockIdx.x;
  double acc = 0.0;
  for (int k = threadIdx.x; k < cols; k += 256) {
    const double v = (double)bf16_to_f32(w[(size_t)r * cols + k]);
    acc += v * v;
  }
  ssum[threadIdx.x] = acc;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) ssum[threadIdx.x] += ssum[threadIdx.x + s];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    rowexp[r] = 0;
    atomicMax(&trailer->max_row_norm_bits, (unsigned long long)__double_as_longlong(sqrt(ssum[0])));
  }
}

// Exponent dword of lane l of block (t, sb): byte j = E5 << 2 of the lane's group in K-step j.
__device__ __forceinline__ uint32_t lane_exponents(const uint8_t* e8, int cols, int row, int sb, int qq,
                                                   const int* rowexp) {
  const int groups = cols / 16;
  const int base = rowexp[row] + 132;
  uint32_t dw = 0;
  for (int jj = 0; jj < kSteps; ++jj) {
    const int e = e8[(size_t)row * groups + sb * 16 + jj * 4 + qq];
    const int e5 = e - base + 20;
    dw |= ((e && e5 >= 1) ? (uint32_t)(e5 << 2) : 0u) << (8 * jj);
  }
  return dw;
}

// One thread per (block u, K-step j, lane l): 16 mantissa bytes; j == 0 threads also write the
// lane's exponent dword.
__global__ void pack_bfp8_kernel(const int8_t* __restrict__ q, const uint8_t* __restrict__ e8,
                                 int rows, int cols, const int* __restrict__ rowexp,
                                 uint8_t* __restrict__ packed) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int j = (int)((tid >> 6) & 3);
  const long u = tid >> 8;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int r = l & 15, qq = l >> 4;
  const int row = t * kTileRows + r;
  const int k0 = sb * kSuperK + j * 64 + qq * 16;
  const u32x4 src = *(const u32x4*)(q + (size_t)row * cols + k0);
  uint8_t* blk = packed + (size_t)u * kBfp8Block;
  *(u32x4*)(blk + j * 1024 + l * 16) = src ^ u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
  if (j == 0) *(uint32_t*)(blk + 4096 + l * 4) = lane_exponents(e8, cols, row, sb, qq, rowexp);
}

// bf4: one thread per (block u, K-step pair p, lane l): 2 x 16 mantissas -> 16 nibble bytes.
__device__ __forceinline__ uint32_t nibbles8(const int8_t* v) {  // values v[0..7] -> one dword
  uint32_t d = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b)
    d |= ((uint32_t)(v[b] + 8) | ((uint32_t)(v[b + 4] + 8) << 4)) << (8 * b);
  return d;
}

__global__ void pack_bf4_kernel(const int8_t* __restrict__ q, const uint8_t* __restrict__ e8, int rows, int cols,
                                const int* __restrict__ rowexp, uint8_t* __restrict__ packed) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * 2 * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int pp = (int)((tid >> 6) & 1);
  const long u = tid >> 7;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int qq = l >> 4, row = t * kTileRows + (l & 15);
  uint32_t out[4];
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int j = 2 * pp + sub;
    int8_t v[16];
    const int8_t* src = q + (size_t)row * cols + sb * kSuperK + j * 64 + qq * 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = src[i];
    out[2 * sub] = nibbles8(v);
    out[2 * sub + 1] = nibbles8(v + 8);
  }
  uint8_t* blk = packed + (size_t)u * kBf4Block;
  *(u32x4*)(blk + pp * 1024 + l * 16) = u32x4{out[0], out[1], out[2], out[3]};
  if (pp == 0) *(uint32_t*)(blk + 2048 + l * 4) = lane_exponents(e8, cols, row, sb, qq, rowexp);
}

// Inverse of pack_bf4_kernel (same thread mapping).
__global__ void unpack_bf4_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                  const int* __restrict__ rowexp, int8_t* __restrict__ q, uint8_t* __restrict__ e8) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * 2 * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int pp = (int)((tid >> 6) & 1);
  const long u = tid >> 7;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int qq = l >> 4, row = t * kTileRows + (l & 15);
  const uint8_t* blk = packed + (size_t)u * kBf4Block;
  const u32x4 m = *(const u32x4*)(blk + pp * 1024 + l * 16);
  const uint32_t dw = *(const uint32_t*)(blk + 2048 + l * 4);
  const int base = rowexp[row] + 132;
#pragma unroll
  for (int sub = 0; sub < 2; ++sub) {
    const int j = 2 * pp + sub;
    int8_t* dst = q + (size_t)row * cols + sb * kSuperK + j * 64 + qq * 16;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t d = m[2 * sub + h];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        dst[8 * h + b] = (int8_t)((int)((d >> (8 * b)) & 0xfu) - 8);
        dst[8 * h + b + 4] = (int8_t)((int)((d >> (8 * b + 4)) & 0xfu) - 8);
      }
    }
    const int e5 = (int)((dw >> (8 * j)) & 0xffu) >> 2;
    e8[(size_t)row * (cols / 16) + sb * 16 + j * 4 + qq] = (uint8_t)(e5 ? e5 - 20 + base : 0);
  }
}

// Audit dequantiser for bf4: the GEMM's dq16_bf4 routine, then the row scale.
__global__ void dequant_bf4_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                   const int* __restrict__ rowexp, float* __restrict__ out) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int j = (int)((tid >> 6) & 3);
  const long u = tid >> 8;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int row = t * kTileRows + (l & 15), qq = l >> 4;
  const uint8_t* blk = packed + (size_t)u * kBf4Block;
  const u32x2 m = *(const u32x2*)(blk + (j >> 1) * 1024 + l * 16 + (j & 1) * 8);
  const uint32_t dw = *(const uint32_t*)(blk + 2048 + l * 4);
  f16x8 a0, a1;
  dq16_bf4(m.x, m.y, scale_pair(dw, j), a0, a1);
  const int re = rowexp[row];
  float* o = out + (size_t)row * cols + sb * kSuperK + j * 64 + qq * 16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] = __builtin_amdgcn_ldexpf((float)a0[i], re);
    o[8 + i] = __builtin_amdgcn_ldexpf((float)a1[i], re);
  }
}

// One thread per (block, K-step, half, lane): 8 bf16 values (16 bytes).
__global__ void pack_bf16_kernel(const uint16_t* __restrict__ w, int rows, int cols,
                                 uint8_t* __restrict__ packed) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 2 * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int h = (int)((tid >> 6) & 1);
  const int j = (int)((tid >> 7) & 3);
  const long u = tid >> 9;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int row = t * kTileRows + (l & 15);
  const int k0 = sb * kSuperK + j * 64 + (l >> 4) * 16 + h * 8;
  *(u32x4*)(packed + (size_t)u * kBf16Block + j * 2048 + h * 1024 + l * 16) =
      *(const u32x4*)(w + (size_t)row * cols + k0);
}

// Inverse of pack_bfp8_kernel (same thread mapping).
__global__ void unpack_bfp8_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                   const int* __restrict__ rowexp, int8_t* __restrict__ q,
                                   uint8_t* __restrict__ e8) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int j = (int)((tid >> 6) & 3);
  const long u = tid >> 8;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int row = t * kTileRows + (l & 15), qq = l >> 4;
  const uint8_t* blk = packed + (size_t)u * kBfp8Block;
  const u32x4 m = *(const u32x4*)(blk + j * 1024 + l * 16);
  *(u32x4*)(q + (size_t)row * cols + sb * kSuperK + j * 64 + qq * 16) =
      m ^ u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u};
  const uint32_t dw = *(const uint32_t*)(blk + 4096 + l * 4);
  const int e5 = (int)((dw >> (8 * j)) & 0xffu) >> 2;
  const int base = rowexp[row] + 132;
  e8[(size_t)row * (cols / 16) + sb * 16 + j * 4 + qq] = (uint8_t)(e5 ? e5 - 20 + base : 0);
}

// Audit dequantiser: the GEMM's dq16 routine, then the row scale.
__global__ void dequant_bfp8_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                    const int* __restrict__ rowexp, float* __restrict__ out) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int j = (int)((tid >> 6) & 3);
  const long u = tid >> 8;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int row = t * kTileRows + (l & 15), qq = l >> 4;
  const uint8_t* blk = packed + (size_t)u * kBfp8Block;
  const u32x4 m = *(const u32x4*)(blk + j * 1024 + l * 16);
  const uint32_t dw = *(const uint32_t*)(blk + 4096 + l * 4);
  f16x8 a0, a1;
  dq16(m, scale_pair(dw, j), a0, a1);
  const int re = rowexp[row];
  float* o = out + (size_t)row * cols + sb * kSuperK + j * 64 + qq * 16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] = __builtin_amdgcn_ldexpf((float)a0[i], re);
    o[8 + i] = __builtin_amdgcn_ldexpf((float)a1[i], re);
  }
}

__global__ void dequant_bf16_kernel(const uint8_t* __restrict__ packed, int rows, int cols,
                                    float* __restrict__ out) {
  const int C = cols / kSuperK;
  const long tid = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long total = (long)(rows / kTileRows) * C * kSteps * 2 * 64;
  if (tid >= total) return;
  const int l = (int)(tid & 63);
  const int h = (int)((tid >> 6) & 1);
  const int j = (int)((tid >> 7) & 3);
  const long u = tid >> 9;
  const int t = (int)(u / C), sb = (int)(u % C);
  const int row = t * kTileRows + (l & 15);
  const int k0 = sb * kSuperK + j * 64 + (l >> 4) * 16 + h * 8;
  const u32x4 v = *(const u32x4*)(packed + (size_t)u * kBf16Block + j * 2048 + h * 1024 + l * 16);
  float* o = out + (size_t)row * cols + k0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[2 * i] = bf16_to_f32((uint16_t)(v[i] & 0xffffu));
    o[2 * i + 1] = bf16_to_f32((uint16_t)(v[i] >> 16));
  }
}

__global__ void fill_zero_kernel(u32x4* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------- host launchers

static inline unsigned blocks_for(long n, int threads) { return (unsigned)((n + threads - 1) / threads); }

int launch_quantize(const void* w, int rows, int cols, void* q, void* e8, uint32_t* bad, int mbits, hipStream_t s) {
  const long n = (long)rows * (cols / 16);
  if (mbits == 3)
    hipLaunchKernelGGL(quantize_kernel<3>, dim3(blocks_for(n, 256)), dim3(256), 0, s, (const uint16_t*)w, rows, cols,
                       (int8_t*)q, (uint8_t*)e8, bad);
  else
    hipLaunchKernelGGL(quantize_kernel<7>, dim3(blocks_for(n, 256)), dim3(256), 0, s, (const uint16_t*)w, rows, cols,
                       (int8_t*)q, (uint8_t*)e8, bad);
  return check_launch("quantize_kernel");
}

int launch_pack(const void* src0, const void* src1, int rows, int cols, int fmt, void* packed, hipStream_t s) {
  uint8_t* base = (uint8_t*)packed;
  int* rowexp = (int*)(base + rowexp_offset(rows, cols, fmt));
  Trailer* tr = (Trailer*)(base + trailer_offset(rows, cols, fmt));
  hipLaunchKernelGGL(trailer_init_kernel, dim3(1), dim3(64), 0, s, tr);
  if (fmt == 1 || fmt == 2) {
    hipLaunchKernelGGL(rowinfo_bfp8_kernel, dim3(rows), dim3(256), 0, s, (const int8_t*)src0,
                       (const uint8_t*)src1, rows, cols, rowexp, tr);
    if (fmt == 1) {
      const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 64;
      hipLaunchKernelGGL(pack_bfp8_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, (const int8_t*)src0,
                         (const uint8_t*)src1, rows, cols, (const int*)rowexp, base);
    } else {
      const long n = (long)(rows / kTileRows) * (cols / kSuperK) * 2 * 64;
      hipLaunchKernelGGL(pack_bf4_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, (const int8_t*)src0,
                         (const uint8_t*)src1, rows, cols, (const int*)rowexp, base);
    }
  } else {
    hipLaunchKernelGGL(rowinfo_bf16_kernel, dim3(rows), dim3(256), 0, s, (const uint16_t*)src0, rows, cols,
                       rowexp, tr);
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 2 * 64;
    hipLaunchKernelGGL(pack_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, (const uint16_t*)src0, rows,
                       cols, base);
  }
  return check_launch("pack kernels");
}

int launch_unpack(const void* packed, int rows, int cols, int fmt, void* q, void* e8, hipStream_t s) {
  const uint8_t* base = (const uint8_t*)packed;
  const int* rowexp = (const int*)(base + rowexp_offset(rows, cols, fmt));
  if (fmt == 2) {
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * 2 * 64;
    hipLaunchKernelGGL(unpack_bf4_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, base, rows, cols, rowexp,
                       (int8_t*)q, (uint8_t*)e8);
  } else {
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 64;
    hipLaunchKernelGGL(unpack_bfp8_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, base, rows, cols, rowexp,
                       (int8_t*)q, (uint8_t*)e8);
  }
  return check_launch("unpack kernel");
}

int launch_dequant(const void* packed, int rows, int cols, int fmt, float* out, hipStream_t s) {
  const uint8_t* base = (const uint8_t*)packed;
  if (fmt == 1) {
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 64;
    hipLaunchKernelGGL(dequant_bfp8_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, base, rows, cols,
                       (const int*)(base + rowexp_offset(rows, cols, 1)), out);
  } else if (fmt == 2) {
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 64;
    hipLaunchKernelGGL(dequant_bf4_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, base, rows, cols,
                       (const int*)(base + rowexp_offset(rows, cols, 2)), out);
  } else {
    const long n = (long)(rows / kTileRows) * (cols / kSuperK) * kSteps * 2 * 64;
    hipLaunchKernelGGL(dequant_bf16_kernel, dim3(blocks_for(n, 256)), dim3(256), 0, s, base, rows, cols, out);
  }
  return check_launch("dequant kernels");
}

int launch_fill_zero(void* p, size_t bytes, hipStream_t s) {
  const size_t n16 = bytes / 16;
  if (n16) {
    unsigned blocks = (unsigned)((n16 + 255) / 256);
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(blocks), dim3(256), 0, s, (u32x4*)p, n16);
  }
  return check_launch("fill_zero_kernel");
}

}  // namespace qmlp
