// qmlp_common.h -- layout constants and device helpers shared by the gfx950 kernels.
//
// Packed ("tiled") weight layout, one matrix W[rows, K] (rows = output features):
//   * 16-row tiles x 256-K superblocks, block index u = tile * (K/256) + superblock (tile-major);
//   * bfp8 block (4352 B): 4 K-steps x 1024 B of excess-128 mantissas, then 256 B of exponents.
//     In K-step j, lane l (row r = l%16, quarter q = l/16) owns bytes [j*1024 + 16l, +16): the
//     mantissas u = q8 + 128 of K = 256*sb + 64*j + 16*q + (0..15) of row r (one 16-value group).
//     Exponent dword of lane l (bytes 4096 + 4l): byte j = E5 << 2, the high byte of the IEEE half
//     2^(E5-15) that scales that group (0 = all-zero group).
//   * bf16 block (8192 B): per K-step two 1 KB halves; lane l owns values 0..7 of its 16 at
//     j*2048 + 16l and values 8..15 at j*2048 + 1024 + 16l.
//   * bf4 block (2304 B): 4-bit mantissas u = q + 8 (q in [-7, 7]); K-step j of lane l takes 8
//     bytes at 1024*(j/2) + 16l + 8*(j%2): byte b of the first dword is u_b | u_{b+4} << 4, of the
//     second u_{8+b} | u_{12+b} << 4; then the 256 exponent bytes as for bfp8, at 2048.
//   * after the blocks: int32 rowexp[rows] (true weight = (u-128) * 2^(E5-15) * 2^rowexp), then a
//     256-byte trailer {double max_row_norm; uint32 flushed_groups; uint32 magic}.
// One 16x16x32 matrix-core product consumes, per lane, 8 consecutive K values of one weight row
// (A operand) and the same 8 K values of one token row (B operand); the K order inside a lane is
// free as long as A and B agree, which the layout above guarantees.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qmlp {

constexpr int kTileRows = 16;
constexpr int kSuperK = 256;
constexpr int kSteps = 4;
constexpr int kBfp8Block = kSteps * 1024 + 256;  // 4352
constexpr int kBf4Block = kSteps * 512 + 256;     // 2304
constexpr int kBf16Block = kSteps * 2048;        // 8192
constexpr int kTrailer = 256;
constexpr uint32_t kTrailerMagic = 0x514d4c50u;  // "PLMQ"

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct Trailer {
  unsigned long long max_row_norm_bits;  // IEEE double bits (non-negative, so integer max works)
  uint32_t flushed_groups;
  uint32_t magic;
};

__host__ __device__ inline size_t tiles_bytes(int rows, int cols, int fmt) {
  return (size_t)(rows / kTileRows) * (size_t)(cols / kSuperK) *
         (fmt == 1 ? kBfp8Block : (fmt == 2 ? kBf4Block : kBf16Block));
}
__host__ __device__ inline size_t rowexp_offset(int rows, int cols, int fmt) { return tiles_bytes(rows, cols, fmt); }
__host__ __device__ inline size_t trailer_offset(int rows, int cols, int fmt) {
  return tiles_bytes(rows, cols, fmt) + (size_t)rows * 4;
}
__host__ __device__ inline size_t packed_total(int rows, int cols, int fmt) {
  return trailer_offset(rows, cols, fmt) + kTrailer;
}

// ---------------------------------------------------------------- scalar conversions

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Round-to-nearest-even fp32 -> bf16 (quiet NaN kept), the same word arithmetic as torch's cast.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t w = __float_as_uint(f);
  if ((w & 0x7f800000u) == 0x7f800000u && (w & 0x007fffffu)) return (uint16_t)((w >> 16) | 0x40u);
  return (uint16_t)((w + 0x7fffu + ((w >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

// silu(g) * u = g * u / (1 + e^-g) from the hardware base-2 exponential and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each): a few fp32 ulp from the correctly rounded value,
// far below the single fp16 / bf16 rounding of h that follows, in ~8 instructions instead of
// the ~33 of a libm exponential and an IEEE division.  For g below about -88, e^-g is +inf and
// the result -0 (|silu(g)| < 1e-36 there).
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);  // e^-g = 2^(-g log2 e)
  return g * __builtin_amdgcn_rcpf(1.0f + e) * u;
}

// ---------------------------------------------------------------- memory helpers

template <typename T>
__device__ __forceinline__ T ld_stream(const T* p) {  // streamed once: do not keep in cache
  return __builtin_nontemporal_load(p);
}

// s_waitcnt operand: vector memory counter 0, export and LDS/scalar counters not waited on.
constexpr int kWaitVmcnt0 = 0x0f70;

// Partial sums cross workgroups (and XCDs) through device-coherent 16-byte buffer stores and loads
// (the sc1 cache policy of agent-scope atomic accesses, on whole 16-byte lanes so that one
// instruction writes or reads whole lines): coherent at the device level by themselves, so
// publishing needs no L2 write-back and reading no L2 invalidation -- only the wait for the stores
// before the arrival counter moves.  The descriptor's extent bounds every access.
constexpr int kCoherent = 16;                 // buffer cache-policy operand: sc1
constexpr int kBufferRsrcWord3 = 0x00020000;  // raw (untyped) buffer descriptor, gfx9
__device__ __forceinline__ void store_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCoherent);
}
__device__ __forceinline__ f32x4 load_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherent));
}
// Waits until this thread's global loads and stores have completed.  A workgroup barrier does not
// wait for global stores, so every thread calls this before the barrier that precedes an arrival
// counter: the counter then moves only after the stores it announces are visible device-wide.
__device__ __forceinline__ void wait_stores() { __builtin_amdgcn_s_waitcnt(kWaitVmcnt0); }

// ---------------------------------------------------------------- bfp8 in-register dequant
//
// Mantissa byte u (excess-128) and the byte-permute constant 0x64 form the half 0x64uu = 1024+u.
// One packed fma  (1024+u)*s + (-1152*s) = (u-128)*s  gives the exact dequantised half for
// s = 2^(E5-15) with E5 in [1, 20] (|value| <= 127*32, every product and sum exactly representable).

__device__ __forceinline__ f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Scale pair (s, s) of K-step j from the lane's exponent dword.
__device__ __forceinline__ f16x2 scale_pair(uint32_t edw, int j) {
  // perm selector bytes, low to high: 0x0c (constant 0x00), j (exponent byte j of src1), 0x0c, j.
  const uint32_t sel = 0x000c000cu | ((uint32_t)j << 24) | ((uint32_t)j << 8);
  return as_f16x2(__builtin_amdgcn_perm(0u, edw, sel));
}

// Dequantise 4 mantissa bytes -> 4 halves (two f16x2, K order preserved).
__device__ __forceinline__ void dq4(uint32_t w, f16x2 s, f16x2 c, f16x2& lo, f16x2& hi) {
  const f16x2 m0 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u));
  const f16x2 m1 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, w, 0x04030402u));
  lo = __builtin_elementwise_fma(m0, s, c);
  hi = __builtin_elementwise_fma(m1, s, c);
}

// 16 mantissas of one lane (one K-step) -> two 8-half operands (values 0..7 and 8..15).
__device__ __forceinline__ void dq16(u32x4 w, f16x2 s, f16x8& a0, f16x8& a1) {
  const f16x2 c = s * f16x2{(_Float16)-1152.0f, (_Float16)-1152.0f};
  f16x2 p0, p1, p2, p3, p4, p5, p6, p7;
  dq4(w.x, s, c, p0, p1);
  dq4(w.y, s, c, p2, p3);
  dq4(w.z, s, c, p4, p5);
  dq4(w.w, s, c, p6, p7);
  a0 = f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  a1 = f16x8{p4.x, p4.y, p5.x, p5.y, p6.x, p6.y, p7.x, p7.y};
}

// One lane's weights of one K-step, per format WF (0 bf16: two of these, 1 bfp8: 16 bytes,
// 2 bf4: 8 bytes).
template <int WF>
struct StepWord {
  typedef u32x4 type;
};
template <>
struct StepWord<2> {
  typedef u32x2 type;
};

// bf4: the lane's 16 nibbles of one K-step (two dwords) -> two f16x8 operands, exactly
// ((1024 + u) * s - 1032 * s = (u - 8) * s).
__device__ __forceinline__ void dq16_bf4(uint32_t d0, uint32_t d1, f16x2 s, f16x8& a0, f16x8& a1) {
  const f16x2 c = s * f16x2{(_Float16)-1032.0f, (_Float16)-1032.0f};
  f16x2 p0, p1, p2, p3, p4, p5, p6, p7;
  dq4(d0 & 0x0f0f0f0fu, s, c, p0, p1);
  dq4((d0 >> 4) & 0x0f0f0f0fu, s, c, p2, p3);
  dq4(d1 & 0x0f0f0f0fu, s, c, p4, p5);
  dq4((d1 >> 4) & 0x0f0f0f0fu, s, c, p6, p7);
  a0 = f16x8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
  a1 = f16x8{p4.x, p4.y, p5.x, p5.y, p6.x, p6.y, p7.x, p7.y};
}

// bf4 -> two bf16 x8 operands, exactly ((u - 8) * s has at most 4 significant bits).
__device__ __forceinline__ void dq16_bf4_bf16(uint32_t d0, uint32_t d1, uint32_t ebyte, bf16x8& a0, bf16x8& a1) {
  const float s = __uint_as_float(((ebyte >> 2) + 112u) << 23);
  const float c = -8.0f * s;
  uint32_t o[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t d = h ? d1 : d0;
#pragma unroll
    for (int b = 0; b < 2; ++b) {  // values 2b, 2b+1 (low nibbles) and 4+2b, 5+2b (high nibbles)
      const float f0 = __builtin_fmaf((float)((d >> (16 * b)) & 0xfu), s, c);
      const float f1 = __builtin_fmaf((float)((d >> (16 * b + 8)) & 0xfu), s, c);
      const float f4 = __builtin_fmaf((float)((d >> (16 * b + 4)) & 0xfu), s, c);
      const float f5 = __builtin_fmaf((float)((d >> (16 * b + 12)) & 0xfu), s, c);
      o[4 * h + b] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
      o[4 * h + 2 + b] = __builtin_amdgcn_perm(__float_as_uint(f5), __float_as_uint(f4), 0x07060302u);
    }
  }
  a0 = __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
  a1 = __builtin_bit_cast(bf16x8, u32x4{o[4], o[5], o[6], o[7]});
}

// The same 16 mantissas -> two bf16 x8 operands, exactly: (u - 128) * s has at most 8 significant
// bits, s = 2^(E5 - 15) from the exponent byte E5 << 2 (group scale before the row exponent).
__device__ __forceinline__ void dq16_bf16(u32x4 w, uint32_t ebyte, bf16x8& a0, bf16x8& a1) {
  const float s = __uint_as_float(((ebyte >> 2) + 112u) << 23);
  const float c = -128.0f * s;
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t d = w[i];
    const float f0 = __builtin_fmaf((float)(d & 0xffu), s, c);
    const float f1 = __builtin_fmaf((float)((d >> 8) & 0xffu), s, c);
    const float f2 = __builtin_fmaf((float)((d >> 16) & 0xffu), s, c);
    const float f3 = __builtin_fmaf((float)(d >> 24), s, c);
    o[2 * i] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);  // high halves
    o[2 * i + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  }
  a0 = __builtin_bit_cast(bf16x8, u32x4{o[0], o[1], o[2], o[3]});
  a1 = __builtin_bit_cast(bf16x8, u32x4{o[4], o[5], o[6], o[7]});
}

// LDS layout of the matrix-core B operand, 2 KB per 64-K step of 16 token rows.  Lane
// l = 16 q + rr needs K = 16 q + 8 h + (0..7) of token row rr for its two products (h = 0, 1).
// The halves live in separate 1 KB blocks and inside a block the lane's 16-byte slot is
// rr ^ (2 q + h), so that the 8 chunks which fill one token row's step land in distinct 16-byte
// bank groups.  Measured on gfx950 (a probe of 16-byte LDS reads and stores, 16 waves per CU):
// the 64-lane reads of this layout run at ~222 B/clk per CU, as lane-linear reads do, and the
// staging stores at ~75 B/clk.  A rotation by 2 q + h instead of the xor halves the read rate
// (~124 B/clk: lanes 0-15 and 16-31 must address their 256-byte rows alike up to the low two
// slot bits), and no swizzle at all quarters the store rate (~16 B/clk).
__host__ __device__ inline uint32_t bfrag_off(int q, int rr, int h) {
  return (uint32_t)(h * 1024 + (q * 16 + (rr ^ (2 * q + h))) * 16);
}

// Logical workgroup index so that consecutive logical indices share an XCD (hardware dispatches
// workgroup b to XCD b % 8): each XCD then streams one contiguous eighth of the weights and
// neighbouring workgroups that share a tile exchange partial sums through the same L2.
__device__ __forceinline__ int xcd_logical(int b, int P) {
  if (P % 8) return b;
  return (b % 8) * (P / 8) + b / 8;
}

}  // namespace qmlp
