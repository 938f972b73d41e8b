// qmlp_gemv.hip -- weight-streaming kernels for M <= 32 tokens (decode / speculative verify).
//
// Reference realisation being replaced: FusedProjection (scripts/ci/fused_1d.py:96-196: 91
// workers x 3 gate/up tile pairs, activation multicast fused_1d_input.cpp:1-51, weight reader
// fused_1d_weights.cpp:1-44, SiLU*mul epilogue) followed by the widened down projection
// (scripts/ci/mlp_down_grid.py:4-12).
//
// Work split.  A projection W[N, K] is T = N/16 row tiles x C = K/256 superblocks of 256 K values.
// The (tile, superblock) grid is cut into Ng tile groups (G tiles each) x S K-splits (split q
// covers superblocks [q*C/S, (q+1)*C/S), at most KQ = ceil(C/S)), one workgroup per rectangle,
// P = Ng * S <= #CUs workgroups with (nearly) equal work.  The M tokens form MG = 1 or 2 groups
// of 16, one 16x16 matrix-core output tile each: every dequantised weight fragment feeds MG
// products.  At the Qwen3-27B shape:
//   16 tokens: gate/up 121 groups of 9 tiles x 2 halves of 10 superblocks (242 workgroups of 90
//              units), down 64 groups of 5 tiles x 4 quarters of 17 (256 workgroups of 85 units);
//   32 tokens: gate/up 64 groups of 17 tiles x 4 quarters of 5 superblocks (256 workgroups of 85
//              units), down 32 groups of 10 tiles x 8 eighths of 8 or 9 (256 x at most 90 units).
//
// Inside a workgroup:
//   1. the token activations of its K range are staged once into LDS in the matrix-core B
//      operand order (block-float weights: converted bf16 -> fp16 with a per-(token, K range)
//      power of two);
//   2. the 8 waves split the rectangle's units (tile-major) into equal contiguous ranges and
//      stream their weight blocks (register stages, non-temporal 16-byte loads), dequantising in
//      registers; a wave's partial sums are parked in registers at tile boundaries;
//   3. after the loop the parked partials go to LDS (over the staged activations, no longer
//      needed), each tile's partials are summed in wave order and published to a workspace slot;
//      each thread waits for its stores, then one arrival counter per workgroup;
//   4. the last of the S workgroups of a tile group sums the S slots in K order (deterministic)
//      and runs the epilogue: gate/up -> h = silu(g) * u (bf16, or fp16 * 2^th for block-float
//      weights), down -> out = residual + y (bf16 or fp32).  It resets the counter for the next call.
#include <algorithm>
#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <utility>

#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

struct GvParams {
  const uint8_t* w0;
  const uint8_t* w1;
  const int* rowexp0;
  const int* rowexp1;
  const uint16_t* src;  // activations [M, K] row-major: x (bf16) for gate/up, h for down
  int M, K, N;
  int C, T, G, S, KQ, Ng, P, maxseg;  // KQ: superblocks of the longest K split
  int x_scale;            // 1: src is bf16 and is converted to fp16 * 2^t (block-float gate/up)
  const uint16_t* normw;  // gate/up with the RMSNorm prologue: bf16 [K] weight w (gain 1 + w)
  float eps;              //   and its epsilon
  const int* th_in;       // block-float down: h = h16 * 2^-th[m]
  int* th_out;            // block-float gate/up: th[m] written by tile group 0
  const Trailer* tg;      // block-float gate/up: weight row-norm trailers for the h bound
  const Trailer* tu;
  void* out;              // gate/up: h [M, N] 16-bit; down: out [M, N] bf16 or fp32
  const void* residual;   // down: [M, N] bf16 or fp32, may alias out
  int out_f32, res_f32;
  float* part;            // [P][G][NMAT * MG * 64] f32x4 partial slots
  float* pss;             // [P][kPssStride] per-workgroup token sums of the staged values' squares
                          // (h bound)
  int* counters;          // [Ng] arrival counters (left at zero)
};

constexpr int kPssStride = 64;  // floats of token sums per workgroup

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Per-(matrices, token groups) constants.  Both bound the registers of one wave to ~48 VGPRs:
//   kMaxSeg: parked partial tiles per wave (the planner rejects splits that need more);
//   kQb:     K splits whose partials the last arrival requests in its first batch.
template <int NMAT, int MG>
struct GvTune {
  static constexpr int kMaxSeg = 12 / (NMAT * MG);
  static constexpr int kQb = (NMAT == 2 ? 2 : 4) * MG;
};

// First superblock of K split q (split lengths differ by at most one superblock).  q * C stays
// far below 2^31 (C = K / 256 and q < S <= 16), so 32-bit arithmetic suffices.
__host__ __device__ inline int split_start(int q, int C, int S) { return q * C / S; }

// WF: 0 bf16, 1 bfp8, 2 bf4 weights.  A bf4 register holds two K-steps of the lane.
template <int WF, int NMAT, int SPS>
struct GStage {
  u32x4 w[NMAT][WF == 2 ? SPS / 2 : SPS][WF ? 1 : 2];
  uint32_t e[NMAT];
};

// ---------------------------------------------------------------- staging of the B operand
//
// LDS layout: for each K-step kk of the workgroup's K range and token group mg, 2 KB at
// (kk * MG + mg) * 2 KB in bfrag_off order (lane l = 16 * quarter + m reads the 16 values
// K = 64 kk + 16 quarter + (0..15) of token row 16 mg + m as two conflict-free 16-byte loads).
//
// Staging is split in two so that the activation loads are issued before the first weight
// loads (vector loads complete in order: waiting for activations issued after the weights would
// also wait for the weights).  Thread (m = token row, tl) handles chunks of 8 values at
// K = 8 * (tl + c * TPR), c < nch = kq * MG; all MAXCH loads are unconditional (clamped chunk index).
template <int MAXCH, bool NORM>
struct BStage {
  u32x4 v[MAXCH];
  u32x4 w[NORM ? MAXCH : 1];  // RMSNorm weight of the same K values
};

template <int NW, int MAXCH, bool NORM, int MG>
__device__ __forceinline__ void stage_b_issue(const GvParams& p, int k0, int kq, BStage<MAXCH, NORM>& bs) {
  constexpr int TPR = NW * 64 / (16 * MG);  // threads per token row
  const int m = threadIdx.x / TPR, tl = threadIdx.x % TPR;
  const int mr = min(m, p.M - 1);  // rows beyond M duplicate row M-1 (their outputs are discarded)
  const int nch = kq * kSuperK / (TPR * 8);
  const uint16_t* row = p.src + (size_t)mr * p.K + k0;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) bs.v[c] = *(const u32x4*)(row + (tl + min(c, nch - 1) * TPR) * 8);
  if constexpr (NORM) {
#pragma unroll
    for (int c = 0; c < MAXCH; ++c) bs.w[c] = *(const u32x4*)(p.normw + k0 + (tl + min(c, nch - 1) * TPR) * 8);
  }
}

// Whole-row sum of squares of token row m (RMSNorm prologue): the TPR threads of the row read it
// in 16-byte chunks, kNormBatch loads in flight, and reduce in a fixed order, so every workgroup
// -- whatever its K range -- computes the same value for the same row.
constexpr int kNormBatch = 8;
template <int TPR>
__device__ __forceinline__ float row_sum_squares(const GvParams& p, int m, int tl) {
  const int nfull = p.K / (TPR * 8);
  const uint16_t* row = p.src + (size_t)min(m, p.M - 1) * p.K;
  float sx = 0.f;
  for (int j0 = 0; j0 < nfull; j0 += kNormBatch) {
    u32x4 t[kNormBatch];
#pragma unroll
    for (int b = 0; b < kNormBatch; ++b) t[b] = *(const u32x4*)(row + (tl + min(j0 + b, nfull - 1) * TPR) * 8);
#pragma unroll
    for (int b = 0; b < kNormBatch; ++b)
      if (j0 + b < nfull)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16_to_f32((uint16_t)(t[b][i] & 0xffffu)), hi = bf16_to_f32((uint16_t)(t[b][i] >> 16));
          sx = fmaf(lo, lo, sx);
          sx = fmaf(hi, hi, sx);
        }
  }
#pragma unroll
  for (int o = TPR / 2; o > 0; o >>= 1) sx += __shfl_xor(sx, o);
  return sx;
}

// With the RMSNorm prologue the staged value is the normalised activation
// n = bf16(x * rs * (1 + w)), rs = 1 / sqrt(mean(x^2) + eps) over the whole row -- the bf16 tensor
// the decoder's separate norm hands to the MLP (docker/qwen-c2-graft/graft/layer.py:352-357) --
// then converted like any activation.
template <int NW, int MAXCH, bool NORM, int MG>
__device__ __forceinline__ void stage_b_finish(const GvParams& p, int kq, const BStage<MAXCH, NORM>& bs,
                                               uint8_t* ldsb, int* lds_t, float* lds_ss) {
  constexpr int TPR = NW * 64 / (16 * MG);
  const int m = threadIdx.x / TPR, tl = threadIdx.x % TPR;
  const int nch = kq * kSuperK / (TPR * 8);
  auto lds_off = [&](int e) {  // K offset e of token row m inside the workgroup's range
    const int kk = e >> 6, r = e & 63;
    return (kk * MG + (m >> 4)) * 2048 + (int)bfrag_off(r >> 4, m & 15, (r >> 3) & 1);
  };
  if (!p.x_scale && !NORM) {
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
      if (c < nch) *(u32x4*)(ldsb + lds_off((tl + c * TPR) * 8)) = bs.v[c];
    return;
  }
  if constexpr (!NORM) {
    // bf16 x -> fp16 * 2^t on packed 16-bit words: the magnitudes' integer maximum is the
    // maximum value, the sum of squares comes from v_dot2_f32_bf16, and the conversion is
    // fp16 bits = ((|x| bits - ((112 - t) << 7)) << 3) | sign, exact while x * 2^t is a normal
    // half; values below 2^-14 after scaling (2^-28 of the range maximum) are flushed to zero.
    u16x2 mx2 = {0, 0};
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < MAXCH; ++c)
      if (c < nch)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t r = bs.v[c][i];
          mx2 = __builtin_elementwise_max(mx2, __builtin_bit_cast(u16x2, r & 0x7fff7fffu));
          ss = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, r), __builtin_bit_cast(bf16x2, r), ss, false);
        }
    uint32_t mb = max((uint32_t)mx2.x, (uint32_t)mx2.y);
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) {
      mb = max(mb, (uint32_t)__shfl_xor((int)mb, o));
      ss += __shfl_xor(ss, o);
    }
    const float mxf = bf16_to_f32((uint16_t)mb);
    int e2 = 0;
    if (mxf > 0.f) frexpf(mxf, &e2);
    const int t = mxf > 0.f ? min(15 - e2, 112) : 0;
    if (tl == 0) {
      lds_t[m] = t;
      lds_ss[m] = ss;
    }
    const uint32_t dd = (uint32_t)(112 - t) << 7;
    const u16x2 d2 = __builtin_bit_cast(u16x2, dd | (dd << 16));
#pragma unroll
    for (int c = 0; c < MAXCH; ++c) {
      if (c < nch) {
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t r = bs.v[c][i];
          const u16x2 sub = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, r & 0x7fff7fffu), d2);
          o[i] = __builtin_bit_cast(uint32_t, (u16x2)(sub << (u16x2){3, 3})) | (r & 0x80008000u);
        }
        *(u32x4*)(ldsb + lds_off((tl + c * TPR) * 8)) = u32x4{o[0], o[1], o[2], o[3]};
      }
    }
    return;
  }
  float rs = 1.0f;
  if constexpr (NORM) rs = 1.0f / sqrtf(row_sum_squares<TPR>(p, m, tl) / (float)p.K + p.eps);
  auto value = [&](int c, int i, int hi) {
    const float xr = bf16_to_f32((uint16_t)(hi ? bs.v[c][i] >> 16 : bs.v[c][i] & 0xffffu));
    if constexpr (NORM) {
      const float wv = bf16_to_f32((uint16_t)(hi ? bs.w[c][i] >> 16 : bs.w[c][i] & 0xffffu));
      return bf16_to_f32(f32_to_bf16(xr * rs * (1.0f + wv)));
    }
    return xr;
  };
  // block float: value -> fp16 * 2^t with max|value| * 2^t in [2^14, 2^15) over this K range
  // (exact unless a value is 2^31 times smaller than the range maximum).  The range's sum of
  // squares feeds the h bound.
  float mx = 0.f, ss = 0.f;
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    if (c < nch) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int hi = 0; hi < 2; ++hi) {
          const float v = value(c, i, hi);
          mx = fmaxf(mx, fabsf(v));
          ss = fmaf(v, v, ss);
        }
      }
    }
  }
  // reduce over the TPR threads of this row (a fixed tree inside one wave: deterministic)
#pragma unroll
  for (int o = TPR / 2; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    ss += __shfl_xor(ss, o);
  }
  int e2 = 0;
  if (mx > 0.f) frexpf(mx, &e2);
  const int t = (p.x_scale && mx > 0.f) ? 15 - e2 : 0;
  if (tl == 0) {
    lds_t[m] = t;
    lds_ss[m] = ss;
  }
#pragma unroll
  for (int c = 0; c < MAXCH; ++c) {
    if (c < nch) {
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = value(c, i, 0), b = value(c, i, 1);
        if (p.x_scale)
          o[i] = (uint32_t)f32_to_f16_bits(__builtin_amdgcn_ldexpf(a, t)) |
                 ((uint32_t)f32_to_f16_bits(__builtin_amdgcn_ldexpf(b, t)) << 16);
        else
          o[i] = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
      }
      *(u32x4*)(ldsb + lds_off((tl + c * TPR) * 8)) = u32x4{o[0], o[1], o[2], o[3]};
    }
  }
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t part_rsrc(const GvParams& p, int slot_f32x4) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, p.P * p.G * slot_f32x4 * 16, kBufferRsrcWord3);
}

// ---------------------------------------------------------------- main loop pieces

struct GPos {
  int unit, part, tl, s;  // unit within the rectangle, stage part, tile (local), superblock (local)
};

template <int SPU>
__device__ __forceinline__ void gadvance(GPos& q, int kq) {
  if (++q.part == SPU) {
    q.part = 0;
    ++q.unit;
    if (++q.s == kq) {
      q.s = 0;
      ++q.tl;
    }
  }
}

template <int WF, int NMAT, int SPS>
__device__ __forceinline__ void gload(GStage<WF, NMAT, SPS>& st, const GvParams& p, size_t blk_base, const GPos& q,
                                      uint32_t lw, uint32_t le) {
  constexpr int BLK = WF == 2 ? kBf4Block : (WF ? kBfp8Block : kBf16Block);
  const size_t blk = (blk_base + (size_t)q.tl * p.C + q.s) * BLK;
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat) {
    const uint8_t* b = (mat ? p.w1 : p.w0) + blk;
    const uint8_t* bp = b + q.part * SPS * (WF == 2 ? 512 : (WF ? 1024 : 2048));
#pragma unroll
    for (int jj = 0; jj < (WF == 2 ? SPS / 2 : SPS); ++jj) {
      if constexpr (WF) {
        st.w[mat][jj][0] = ld_stream((const u32x4*)(bp + lw + jj * 1024));
      } else {
        st.w[mat][jj][0] = ld_stream((const u32x4*)(bp + lw + jj * 2048));
        st.w[mat][jj][1] = ld_stream((const u32x4*)(bp + lw + jj * 2048 + 1024));
      }
    }
    if constexpr (WF) st.e[mat] = ld_stream((const uint32_t*)(b + le));
  }
}

template <int WF, int NMAT, int SPS, int MG>
__device__ __forceinline__ void gcompute(const GStage<WF, NMAT, SPS>& st, const GPos& q, const uint8_t* ldsb,
                                         int lane, f32x4 (&acc)[NMAT][MG][2]) {
#pragma unroll
  for (int jj = 0; jj < SPS; ++jj) {
    const int j = q.part * SPS + jj;
    const uint8_t* bp = ldsb + (q.s * kSteps + j) * MG * 2048;
    f16x8 b0[MG], b1[MG];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      b0[mg] = *(const f16x8*)(bp + mg * 2048 + bfrag_off(lane >> 4, lane & 15, 0));
      b1[mg] = *(const f16x8*)(bp + mg * 2048 + bfrag_off(lane >> 4, lane & 15, 1));
    }
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      if constexpr (WF) {
        f16x8 a0, a1;
        if constexpr (WF == 2) {
          const u32x4 d = st.w[mat][jj / 2][0];
          dq16_bf4(jj & 1 ? d.z : d.x, jj & 1 ? d.w : d.y, scale_pair(st.e[mat], j), a0, a1);
        } else {
          dq16(st.w[mat][jj][0], scale_pair(st.e[mat], j), a0, a1);
        }
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          acc[mat][mg][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0[mg], acc[mat][mg][0], 0, 0, 0);
          acc[mat][mg][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1[mg], acc[mat][mg][1], 0, 0, 0);
        }
      } else {
        const bf16x8 a0 = __builtin_bit_cast(bf16x8, st.w[mat][jj][0]);
        const bf16x8 a1 = __builtin_bit_cast(bf16x8, st.w[mat][jj][1]);
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          acc[mat][mg][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, __builtin_bit_cast(bf16x8, b0[mg]),
                                                                    acc[mat][mg][0], 0, 0, 0);
          acc[mat][mg][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, __builtin_bit_cast(bf16x8, b1[mg]),
                                                                    acc[mat][mg][1], 0, 0, 0);
        }
      }
    }
  }
}

// ---------------------------------------------------------------- epilogue (last arrival)
//
// Lane l holds rows 4*(l/16) + v (v = 0..3) of token column m = 16 mg + l % 16 -- the 16x16
// matrix-core output layout, one tile per token group mg.

// Operands of one tile's epilogue that do not depend on the other K splits.
template <int NMAT, int MG>
struct EpiIn {
  u32x4 rexp[NMAT];  // block-float: row exponents of the lane's 4 rows
  u32x4 res[MG];     // down: the lane's 4 residual values per token group (bf16 pairs in .x/.y, or fp32)
  int th[MG];        // block-float down: h scale of the lane's tokens
};

template <int WF, int NMAT, int MG>
__device__ __forceinline__ void epi_load(const GvParams& p, int t, int lane, EpiIn<NMAT, MG>& e) {
  const int nb = t * kTileRows + (lane >> 4) * 4;
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
    e.rexp[mat] = WF ? *(const u32x4*)((mat ? p.rowexp1 : p.rowexp0) + nb) : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    const int m = min(mg * 16 + (lane & 15), p.M - 1);  // tokens >= M load token M-1 (outputs discarded)
    e.res[mg] = u32x4{0u, 0u, 0u, 0u};
    e.th[mg] = 0;
    if constexpr (NMAT == 1) {
      if constexpr (WF != 0) e.th[mg] = p.th_in[m];
      if (p.residual) {
        if (p.res_f32) {
          e.res[mg] = *(const u32x4*)((const float*)p.residual + (size_t)m * p.N + nb);
        } else {
          const u32x2 r = *(const u32x2*)((const uint16_t*)p.residual + (size_t)m * p.N + nb);
          e.res[mg] = u32x4{r.x, r.y, 0u, 0u};
        }
      }
    }
  }
}

template <int WF, int NMAT, int MG>
__device__ __forceinline__ void gepilogue(const GvParams& p, int t, const f32x4 (&tot)[NMAT][MG],
                                          const EpiIn<NMAT, MG>& e, int lane, const int (&th)[MG]) {
  const int nb = t * kTileRows + (lane >> 4) * 4;
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) {
    const int m = mg * 16 + (lane & 15);
    if (m >= p.M) continue;
    uint16_t o[4];
    if constexpr (NMAT == 2) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        float g = tot[0][mg][v], u = tot[1][mg][v];
        if constexpr (WF) {
          g = __builtin_amdgcn_ldexpf(g, (int)e.rexp[0][v]);
          u = __builtin_amdgcn_ldexpf(u, (int)e.rexp[1][v]);
        }
        const float hv = silu_mul(g, u);
        // bf16 weights: h is the bf16 operand of the down projection, rounded once like the
        // reference's fused epilogue; bfp8: fp16 * 2^th (one rounding from fp32).
        o[v] = WF ? f32_to_f16_bits(__builtin_amdgcn_ldexpf(hv, th[mg])) : f32_to_bf16(hv);
      }
    } else {
      float y[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        y[v] = tot[0][mg][v];
        if constexpr (WF) y[v] = __builtin_amdgcn_ldexpf(y[v], (int)e.rexp[0][v] - e.th[mg]);
      }
      if (p.residual) {
        if (p.res_f32) {
#pragma unroll
          for (int v = 0; v < 4; ++v) y[v] += __uint_as_float(e.res[mg][v]);
        } else {
          y[0] += bf16_to_f32((uint16_t)(e.res[mg].x & 0xffffu));
          y[1] += bf16_to_f32((uint16_t)(e.res[mg].x >> 16));
          y[2] += bf16_to_f32((uint16_t)(e.res[mg].y & 0xffffu));
          y[3] += bf16_to_f32((uint16_t)(e.res[mg].y >> 16));
        }
      }
      if (p.out_f32) {
        *(f32x4*)((float*)p.out + (size_t)m * p.N + nb) = f32x4{y[0], y[1], y[2], y[3]};
        continue;
      }
#pragma unroll
      for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16(y[v]);
    }
    *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + nb) =
        u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
  }
}

// ---------------------------------------------------------------- kernel

template <int WF, int NMAT, int NW, int MAXCH, bool NORM, int MG>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(GvParams p) {
  constexpr int SPS = WF ? 4 : 2;  // K-steps per register stage
  constexpr int SPU = kSteps / SPS;
  constexpr int SLOT = NMAT * MG * 64;  // f32x4 per parked partial
  constexpr int ROWS = 16 * MG;
  constexpr int MAXSEG = GvTune<NMAT, MG>::kMaxSeg;
  constexpr int QB = GvTune<NMAT, MG>::kQb;
  extern __shared__ __align__(16) uint8_t lds[];
  __shared__ int s_t[ROWS];
  __shared__ float s_ss[ROWS];
  __shared__ int s_last;
  __shared__ int s_seg[NW][2];  // first and last tile of each wave's unit range (empty: 1 > -1)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = xcd_logical(blockIdx.x, p.P);
  const int g = w / p.S, q = w % p.S;
  const int c0 = split_start(q, p.C, p.S), kq = split_start(q + 1, p.C, p.S) - c0;
  const int Gw = min(p.G, p.T - g * p.G);  // tiles in this group
  const int U = Gw * kq;
  const int ua = (int)((long)wave * U / NW), ub = (int)((long)(wave + 1) * U / NW);
  uint8_t* ldsb = lds;         // B operand (main loop)
  f32x4* slots = (f32x4*)lds;  // [NW][maxseg][SLOT] parked partials (after the main loop)
  const size_t blk_base = (size_t)(g * p.G) * p.C + (size_t)c0;
  const uint32_t lw = (uint32_t)lane * 16u, le = (WF == 2 ? 2048u : 4096u) + (uint32_t)lane * 4u;

  // A wave without units still issues its prologue loads (of a valid unit) so that every load
  // before the staging barrier is unconditional.
  const int u0 = ua < ub ? ua : 0;
  GPos cur;
  cur.unit = u0;
  cur.part = 0;
  cur.tl = u0 / kq;
  cur.s = u0 - cur.tl * kq;
  // Three register stages: while stage i is dequantised and multiplied the loads of stages i+1
  // and i+2 are in flight, and stage i+3 is issued right after stage i is consumed.  Two stages
  // are issued between the activation loads and the B staging so that HBM streams while the
  // activations arrive; the third only after them: the activations queue behind every weight
  // request issued before them across the chip, so a smaller first wave of requests returns
  // them sooner (measured: 1.2 us per layer less than issuing all three first).  The
  // steady-state loop only issues unconditional loads (a predicated load would make the
  // compiler wait for every outstanding load); the last <= 5 stages are peeled.
  GStage<WF, NMAT, SPS> s0, s1, s2;
  const int nst = (ub - ua) * SPU;
  GPos P0 = cur, P1 = cur, P2 = cur;
  if (nst > 1) gadvance<SPU>(P1, kq);
  P2 = P1;
  if (nst > 2) gadvance<SPU>(P2, kq);
  BStage<MAXCH, NORM> bs;
  stage_b_issue<NW, MAXCH, NORM, MG>(p, c0 * kSuperK, kq, bs);
  gload(s0, p, blk_base, P0, lw, le);
  gload(s1, p, blk_base, P1, lw, le);  // repeats stage 0 when nst == 1
  stage_b_finish<NW, MAXCH, NORM, MG>(p, kq, bs, ldsb, s_t, s_ss);
  gload(s2, p, blk_base, P2, lw, le);
  __syncthreads();

  // A wave touches consecutive tiles; at each tile boundary its partial sums are parked in
  // registers (pk[0] the latest, shifted with static indices).
  f32x4 pk[MAXSEG][NMAT][MG];
  int npk = 0;
  if (ua < ub) {
    f32x4 acc[NMAT][MG][2];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) acc[mat][mg][0] = acc[mat][mg][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto park = [&]() {
#pragma unroll
      for (int i = MAXSEG - 1; i > 0; --i)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int mg = 0; mg < MG; ++mg) pk[i][mat][mg] = pk[i - 1][mat][mg];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          pk[0][mat][mg] = acc[mat][mg][0] + acc[mat][mg][1];
          acc[mat][mg][0] = acc[mat][mg][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      ++npk;
    };
    int i = 0;
    for (; i + 5 < nst; i += 3) {
      gcompute<WF, NMAT, SPS, MG>(s0, P0, ldsb, lane, acc);
      GPos P3 = P2;
      gadvance<SPU>(P3, kq);
      gload(s0, p, blk_base, P3, lw, le);
      if (P1.tl != P0.tl) park();
      gcompute<WF, NMAT, SPS, MG>(s1, P1, ldsb, lane, acc);
      GPos P4 = P3;
      gadvance<SPU>(P4, kq);
      gload(s1, p, blk_base, P4, lw, le);
      if (P2.tl != P1.tl) park();
      gcompute<WF, NMAT, SPS, MG>(s2, P2, ldsb, lane, acc);
      GPos P5 = P4;
      gadvance<SPU>(P5, kq);
      gload(s2, p, blk_base, P5, lw, le);
      if (P3.tl != P2.tl) park();
      P0 = P3;
      P1 = P4;
      P2 = P5;
    }
    // tail: r = 1..5 stages left; P0..P2 (those that exist) are loaded, P3, P4 are not
    const int r = nst - i;
    GPos P3 = P2, P4 = P2;
    gcompute<WF, NMAT, SPS, MG>(s0, P0, ldsb, lane, acc);
    if (r > 3) {
      gadvance<SPU>(P3, kq);
      gload(s0, p, blk_base, P3, lw, le);
    }
    if (r > 1) {
      if (P1.tl != P0.tl) park();
      gcompute<WF, NMAT, SPS, MG>(s1, P1, ldsb, lane, acc);
      if (r > 4) {
        P4 = P3;
        gadvance<SPU>(P4, kq);
        gload(s1, p, blk_base, P4, lw, le);
      }
      if (r > 2) {
        if (P2.tl != P1.tl) park();
        gcompute<WF, NMAT, SPS, MG>(s2, P2, ldsb, lane, acc);
        if (r > 3) {
          if (P3.tl != P2.tl) park();
          gcompute<WF, NMAT, SPS, MG>(s0, P3, ldsb, lane, acc);
          if (r > 4) {
            if (P4.tl != P3.tl) park();
            gcompute<WF, NMAT, SPS, MG>(s1, P4, ldsb, lane, acc);
          }
        }
      }
    }
    park();
  }
  // The epilogue operands that do not depend on the other K splits (row exponents, residual,
  // h scale, weight norms) are requested now for the first kEpt tiles of each wave -- by every
  // workgroup of the group, as the last arrival is not known yet -- so that the last arrival
  // then waits for a single round trip: the other splits' partial and token sums.
  constexpr int kEpt = 2;
  EpiIn<NMAT, MG> ein[kEpt];
#pragma unroll
  for (int k = 0; k < kEpt; ++k) epi_load<WF, NMAT, MG>(p, g * p.G + min(wave + k * NW, Gw - 1), lane, ein[k]);
  double gn = 0.0, un = 0.0;
  if (p.x_scale) {
    gn = __longlong_as_double((long long)p.tg->max_row_norm_bits);
    un = __longlong_as_double((long long)p.tu->max_row_norm_bits);
  }
  if (lane == 0) {
    s_seg[wave][0] = ua < ub ? ua / kq : 1;
    s_seg[wave][1] = ua < ub ? (ub - 1) / kq : -1;
  }
  __syncthreads();  // every wave is done with the staged activations: their LDS takes the slots

  // parked partials -> LDS slots (slot index = tile - the wave's first tile)
#pragma unroll
  for (int k = 0; k < MAXSEG; ++k) {
    if (k < npk) {
      f32x4* slot = slots + (size_t)(wave * p.maxseg + (npk - 1 - k)) * SLOT;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) slot[(mat * MG + mg) * 64 + lane] = pk[k][mat][mg];
    }
  }
  __syncthreads();

  // publish this workgroup's per-tile partial sums.  Wave w publishes tiles w, w + NW, ... and,
  // if this workgroup arrives last, finishes the same tiles: it keeps the first kEpt of its sums
  // in registers and adds them in place of re-reading its own slots.
  const int m = lane & 15;
  const __amdgpu_buffer_rsrc_t prs = part_rsrc(p, SLOT);
  f32x4 own[kEpt][NMAT][MG];
  auto publish = [&](int tl, f32x4 (&sum)[NMAT][MG]) {
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) sum[mat][mg] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int v = 0; v < NW; ++v) {
      const int vt0 = s_seg[v][0], vt1 = s_seg[v][1];
      if (tl < vt0 || tl > vt1) continue;
      const f32x4* slot = slots + (size_t)(v * p.maxseg + (tl - vt0)) * SLOT;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) sum[mat][mg] += slot[(mat * MG + mg) * 64 + lane];
    }
    if (p.x_scale) {
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) {
        const int t = s_t[mg * 16 + m];
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int v = 0; v < 4; ++v) sum[mat][mg][v] = __builtin_amdgcn_ldexpf(sum[mat][mg][v], -t);
      }
    }
    const uint32_t dst = (uint32_t)((w * p.G + tl) * SLOT + lane) * 16u;
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) store_coherent(prs, dst + (mat * MG + mg) * 1024u, sum[mat][mg]);
  };
#pragma unroll
  for (int k = 0; k < kEpt; ++k)
    if (wave + k * NW < Gw) publish(wave + k * NW, own[k]);
  for (int tl = wave + kEpt * NW; tl < Gw; tl += NW) {
    f32x4 sum[NMAT][MG];
    publish(tl, sum);
  }
  if (p.x_scale && threadIdx.x < ROWS)
    __hip_atomic_store(p.pss + (size_t)w * kPssStride + threadIdx.x, s_ss[threadIdx.x], __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(p.counters + g, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == p.S - 1;
    if (last) __hip_atomic_store(p.counters + g, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last) return;

  // Last arrival.  One batch of loads: the token sums of the first 4 splits (lane 16 j + m holds
  // split j of token 16 mg + m) and the first QB partial slots of each of the wave's first kEpt
  // tiles (indices clamped, so every load is unconditional; the extra copies are not summed).
  // Then the S values of every sum are added in K order (deterministic).
  float ssl[MG];
  auto load_token_sums = [&](int q0) {
    const float* ps = p.pss + (size_t)(g * p.S + min(q0 + (lane >> 4), p.S - 1)) * kPssStride;
#pragma unroll
    for (int mg = 0; mg < MG; ++mg)
      ssl[mg] = __hip_atomic_load(ps + mg * 16 + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  if (p.x_scale) load_token_sums(0);
  auto slot_src = [&](int qq, int tl) {
    return (uint32_t)(((g * p.S + min(qq, p.S - 1)) * p.G + tl) * SLOT + lane) * 16u;
  };
  f32x4 v[kEpt][QB][NMAT][MG];
#pragma unroll
  for (int k = 0; k < kEpt; ++k) {
    const int tl = min(wave + k * NW, Gw - 1);
#pragma unroll
    for (int qq = 0; qq < QB; ++qq) {
      if (qq == q) continue;  // this workgroup's own split: in registers (q is uniform)
      const uint32_t src = slot_src(qq, tl);
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) v[k][qq][mat][mg] = load_coherent(prs, src + (mat * MG + mg) * 1024u);
    }
  }
  int th[MG];
#pragma unroll
  for (int mg = 0; mg < MG; ++mg) th[mg] = 0;
  if (p.x_scale) {
    float ss[MG];
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) ss[mg] = 0.f;
    for (int q0 = 0; q0 < p.S; q0 += 4) {
      if (q0 > 0) load_token_sums(q0);  // more than 4 splits: the next 4 token sums
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int mg = 0; mg < MG; ++mg) {
          const float a = __shfl(ssl[mg], 16 * j + m);
          if (q0 + j < p.S) ss[mg] += a;
        }
    }
#pragma unroll
    for (int mg = 0; mg < MG; ++mg) {
      const double bound = (double)ss[mg] * gn * un * (1.0 + 1.0 / 64.0);
      int eb = 0;
      if (bound > 0.0) frexp(bound, &eb);
      th[mg] = bound > 0.0 ? 15 - eb : 0;
      if (g == 0 && wave == 0 && lane < 16 && mg * 16 + lane < p.M) p.th_out[mg * 16 + lane] = th[mg];
    }
  }
  // slots q0.. of tile tl, added in K order, two splits per round trip (more than QB splits);
  // ow: this workgroup's own sum of the tile, when kept (used in place of its slot)
  auto sum_rest = [&](int tl, int q0, f32x4 (&tot)[NMAT][MG], const f32x4 (*ow)[MG]) {
    for (int qb = q0; qb < p.S; qb += 2) {
      f32x4 u[2][NMAT][MG];
#pragma unroll
      for (int qq = 0; qq < 2; ++qq) {
        const uint32_t src = slot_src(qb + qq, tl);
        const bool mine = ow != nullptr && qb + qq == q;
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int mg = 0; mg < MG; ++mg)
            u[qq][mat][mg] = mine ? ow[mat][mg] : load_coherent(prs, src + (mat * MG + mg) * 1024u);
      }
#pragma unroll
      for (int qq = 0; qq < 2; ++qq)
        if (qb + qq < p.S)
#pragma unroll
          for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
            for (int mg = 0; mg < MG; ++mg) tot[mat][mg] += u[qq][mat][mg];
    }
  };
#pragma unroll
  for (int k = 0; k < kEpt; ++k) {
    const int tl = wave + k * NW;
    if (tl >= Gw) break;
    f32x4 tot[NMAT][MG];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) tot[mat][mg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int qq = 0; qq < QB; ++qq)
      if (qq < p.S)
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int mg = 0; mg < MG; ++mg) tot[mat][mg] += qq == q ? own[k][mat][mg] : v[k][qq][mat][mg];
    sum_rest(tl, QB, tot, own[k]);
    gepilogue<WF, NMAT, MG>(p, g * p.G + tl, tot, ein[k], lane, th);
  }
  // tiles beyond kEpt per wave (groups of more than kEpt * NW tiles)
  for (int tl = wave + kEpt * NW; tl < Gw; tl += NW) {
    EpiIn<NMAT, MG> e;
    epi_load<WF, NMAT, MG>(p, g * p.G + tl, lane, e);
    f32x4 tot[NMAT][MG];
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int mg = 0; mg < MG; ++mg) tot[mat][mg] = f32x4{0.f, 0.f, 0.f, 0.f};
    sum_rest(tl, 0, tot, nullptr);
    gepilogue<WF, NMAT, MG>(p, g * p.G + tl, tot, e, lane, th);
  }
}

// ---------------------------------------------------------------- host side

constexpr int kGemvNW = 8;
constexpr int kGemvMaxChunks = 18;  // B staging chunks per thread (= superblocks per K split x MG)
constexpr int kGemvMaxLds = 160 * 1024 - 1024;  // dynamic LDS; the rest holds the static arrays

static int gemv_max_seg(int nmat, int mg) {
  if (nmat == 2) return mg == 2 ? GvTune<2, 2>::kMaxSeg : GvTune<2, 1>::kMaxSeg;
  return mg == 2 ? GvTune<1, 2>::kMaxSeg : GvTune<1, 1>::kMaxSeg;
}

// The staged activations during the main loop, the parked partials after it (same memory).
static size_t gemv_lds_bytes(const GemvPlan& pl, int nmat, int mg) {
  return std::max((size_t)pl.KQ * kSteps * 2048 * mg, (size_t)kGemvNW * pl.maxseg * nmat * mg * 64 * 16);
}

// Work split: minimise a simple time model over the K split S.  A workgroup streams U = G * KQ
// units (NMAT x 4352-byte blocks each); the last workgroup of a tile group then reads the other
// S - 1 splits' partial tiles per matrix (the model, fitted when it read all S, charges S * G).
// Units cost ~0.16 us per matrix at a CU's share of HBM bandwidth, partial tiles ~0.03 us each
// whatever the token groups (fitted on MI355X to the measured 27B-shape splits: at 16 tokens
// gate/up 2 K splits beat 4, at 32 tokens 4 beat 3, and down 8 beat 10; charging S - 1 picks the
// same splits there); splits using fewer than all CUs pay for it through their larger U.  K
// splits may differ by one superblock.
int plan_gemv(int rows, int K, int nmat, int mg, int num_cus, GemvPlan* out) {
  if (rows <= 0 || K <= 0 || rows % kTileRows || K % kSuperK || (mg != 1 && mg != 2) || (nmat != 1 && nmat != 2))
    return -1;
  const int T = rows / kTileRows, C = K / kSuperK;
  const int cus = num_cus < 1 ? 1 : (num_cus > kMaxWorkgroups ? kMaxWorkgroups : num_cus);
  GemvPlan best{};
  double best_cost = -1.0;
  for (int S = 1; S <= C && S <= kMaxSplit; ++S) {
    const int KQ = (C + S - 1) / S;
    if (KQ * mg > kGemvMaxChunks) continue;  // B staging registers
    const int G = (int)(((long)T * S + cus - 1) / cus);
    const int Ng = (T + G - 1) / G;
    const int P = Ng * S;
    if (P > cus) continue;
    // the most tiles one wave touches, over every workgroup shape (G or the last group's tiles,
    // the shorter or the longer K split)
    int maxseg = 0;
    const int gws[2] = {G, T - (Ng - 1) * G};
    for (int kq = C / S; kq <= KQ; ++kq)
      for (int Gw : gws) {
        const int U = Gw * kq;
        for (int v = 0; v < kGemvNW; ++v) {
          const int ua = (int)((long)v * U / kGemvNW), ub = (int)((long)(v + 1) * U / kGemvNW);
          if (ua < ub) maxseg = std::max(maxseg, (ub - 1) / kq - ua / kq + 1);
        }
      }
    if (maxseg > gemv_max_seg(nmat, mg)) continue;  // parked-partial registers
    GemvPlan c{G, S, KQ, Ng, P, maxseg};
    if (gemv_lds_bytes(c, nmat, mg) > (size_t)kGemvMaxLds) continue;
    const int U = G * KQ;
    const double cost = U * 0.16 * nmat + (S > 1 ? S * G * nmat * 0.03 : 0.0);
    if (best_cost < 0 || cost < best_cost - 1e-9) {
      best = c;
      best_cost = cost;
    }
  }
  if (best_cost < 0) return -2;
  *out = best;
  return 0;
}

// Raises a kernel's dynamic LDS limit to kGemvMaxLds, once per (kernel, device); thread-safe.
static int enable_large_lds(const void* kern, const char* what) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return set_error(-7, "%s: no HIP device", what);
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({kern, dev})) return 0;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, kGemvMaxLds) != hipSuccess)
    return set_error(-4, "%s: cannot enable %d bytes of LDS", what, kGemvMaxLds);
  done.insert({kern, dev});
  return 0;
}

template <int WF, int NMAT, int MAXCH, bool NORM, int MG>
static int launch_gemv_ch(const GvParams& p, size_t lds, hipStream_t s) {
  auto kern = gemv_kernel<WF, NMAT, kGemvNW, MAXCH, NORM, MG>;
  if (int rc = enable_large_lds((const void*)kern, "gemv_kernel")) return rc;
  launch_timed(NMAT == 2 ? 0 : 1, kern, dim3(p.P), dim3(kGemvNW * 64), lds, s, p);
  return check_launch("gemv_kernel");
}

// The staging register array is sized by a small set of buckets (loads beyond KQ * MG are clamped
// duplicates).
template <int WF, int NMAT, bool NORM, int MG>
static int launch_gemv_mg(const GvParams& p, size_t lds, hipStream_t s) {
  const int nch = p.KQ * MG;
  if (nch <= 4) return launch_gemv_ch<WF, NMAT, 4, NORM, MG>(p, lds, s);
  if (nch <= 10) return launch_gemv_ch<WF, NMAT, 10, NORM, MG>(p, lds, s);
  return launch_gemv_ch<WF, NMAT, kGemvMaxChunks, NORM, MG>(p, lds, s);
}

template <int WF, int NMAT, bool NORM = false>
static int launch_gemv(const GvParams& p, int mg, size_t lds, hipStream_t s) {
  return mg == 2 ? launch_gemv_mg<WF, NMAT, NORM, 2>(p, lds, s) : launch_gemv_mg<WF, NMAT, NORM, 1>(p, lds, s);
}

size_t gemv_part_bytes(int rows, int K, int nmat, int mg) {
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, int>, size_t> cache;
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(rows, K, nmat, mg);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  size_t best = 0;
  for (int cus = 1; cus <= kMaxWorkgroups; ++cus) {
    GemvPlan pl;
    if (plan_gemv(rows, K, nmat, mg, cus, &pl) == 0)
      best = std::max(best, (size_t)pl.P * pl.G * nmat * mg * 64 * 16);
  }
  cache[key] = best;
  return best;
}

int gemv_groups(int M) { return M > 16 ? 2 : 1; }

bool gemv_supported(int M, int H, int I, int num_cus) {
  if (M < 1 || M > 32) return false;
  const int mg = gemv_groups(M);
  GemvPlan a, b;
  return plan_gemv(I, H, 2, mg, num_cus, &a) == 0 && plan_gemv(H, I, 1, mg, num_cus, &b) == 0;
}

int launch_forward_gemv(const ForwardArgs& a, int num_cus, hipStream_t s) {
  const WsLayout L = ws_layout(a.M, a.H, a.I, a.fmt);
  const int fmt = a.fmt, mg = gemv_groups(a.M);
  GemvPlan pg, pd;
  if (plan_gemv(a.I, a.H, 2, mg, num_cus, &pg) || plan_gemv(a.H, a.I, 1, mg, num_cus, &pd))
    return set_error(-1, "no weight-streaming split for M=%d H=%d I=%d", a.M, a.H, a.I);
  int* th = (int*)(a.ws + L.th);
  uint16_t* h = (uint16_t*)(a.ws + L.h);
  GvParams g{};
  g.w0 = a.wg;
  g.w1 = a.wu;
  g.rowexp0 = (const int*)(a.wg + rowexp_offset(a.I, a.H, fmt));
  g.rowexp1 = (const int*)(a.wu + rowexp_offset(a.I, a.H, fmt));
  g.src = (const uint16_t*)a.x;
  g.M = a.M;
  g.K = a.H;
  g.N = a.I;
  g.C = a.H / kSuperK;
  g.T = a.I / kTileRows;
  g.G = pg.G;
  g.S = pg.S;
  g.KQ = pg.KQ;
  g.Ng = pg.Ng;
  g.P = pg.P;
  g.maxseg = pg.maxseg;
  g.x_scale = fmt != 0;
  g.normw = (const uint16_t*)a.normw;
  g.eps = a.eps;
  g.th_out = th;
  g.tg = (const Trailer*)(a.wg + trailer_offset(a.I, a.H, fmt));
  g.tu = (const Trailer*)(a.wu + trailer_offset(a.I, a.H, fmt));
  g.out = h;
  g.part = (float*)(a.ws + L.part_gu);
  g.pss = (float*)(a.ws + L.pss);
  g.counters = (int*)(a.ws + L.counters_gu);
  const size_t lg = gemv_lds_bytes(pg, 2, mg);
  int rc;
  if (fmt == 2)
    rc = a.normw ? launch_gemv<2, 2, true>(g, mg, lg, s) : launch_gemv<2, 2>(g, mg, lg, s);
  else if (fmt == 1)
    rc = a.normw ? launch_gemv<1, 2, true>(g, mg, lg, s) : launch_gemv<1, 2>(g, mg, lg, s);
  else
    rc = a.normw ? launch_gemv<0, 2, true>(g, mg, lg, s) : launch_gemv<0, 2>(g, mg, lg, s);
  if (rc) return rc;
  GvParams d{};
  d.w0 = a.wd;
  const int dfmt = down_format(fmt);
  d.rowexp0 = (const int*)(a.wd + rowexp_offset(a.H, a.I, dfmt));
  d.src = h;
  d.M = a.M;
  d.K = a.I;
  d.N = a.H;
  d.C = a.I / kSuperK;
  d.T = a.H / kTileRows;
  d.G = pd.G;
  d.S = pd.S;
  d.KQ = pd.KQ;
  d.Ng = pd.Ng;
  d.P = pd.P;
  d.maxseg = pd.maxseg;
  d.x_scale = 0;
  d.th_in = th;
  d.out = a.out;
  d.residual = a.residual;
  d.out_f32 = a.out_f32;
  d.res_f32 = a.res_f32;
  d.part = (float*)(a.ws + L.part_d);
  d.counters = (int*)(a.ws + L.counters_d);
  const size_t ld = gemv_lds_bytes(pd, 1, mg);
  rc = dfmt == 1 ? launch_gemv<1, 1>(d, mg, ld, s) : launch_gemv<0, 1>(d, mg, ld, s);
  return rc;
}

}  // namespace qmlp
