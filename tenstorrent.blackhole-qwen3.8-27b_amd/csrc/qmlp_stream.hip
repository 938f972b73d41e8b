// qmlp_stream.hip -- weight-streaming kernels for M <= 32 tokens (decode / speculative verify).
//
// Reference realisation being replaced: FusedProjection (scripts/ci/fused_1d.py:96-196: 91
// workers x 3 gate/up tile pairs, activation multicast fused_1d_input.cpp:1-51, weight reader
// fused_1d_weights.cpp:1-44, SiLU*mul epilogue rounded once to bf16, fused_1d.py:10-22) followed
// by the widened down projection (scripts/ci/mlp_down_grid.py:4-12) and the layer's residual add
// (docker/qwen-c2-graft/graft/layer.py:357).
//
// Operands.  Every weight format feeds bf16 matrix-core products with fp32 accumulation: bf16
// weights as they are, bfp8 and bf4 weights dequantised in registers (a mantissa u and its group
// scale s give (u - 128) * s, resp. (u - 8) * s, at most 8 significant bits, so the bf16 value is
// exact).  The tokens are the
// B operand, read by each wave straight from L2 in the matrix-core lane order (token rows are
// small and shared by every workgroup), so no workgroup stages activations and h stays bf16 --
// the reference's own rounding of h.
//
// Work split (stream-K).  A projection W[N, K] is T = N/16 row tiles x 4*C 64-K steps per tile,
// S = 4*T*C steps in tile-major order.  Workgroup w owns steps [w*S/P, (w+1)*S/P), its wave v the
// v-th eighth of that range, so every wave streams the same number of bytes.  A wave accumulates
// in registers and parks its partial sums in LDS whenever its range crosses a tile boundary;
// after one barrier each tile of the workgroup is summed in wave order.  Tiles inside the
// workgroup's range are finished at once; a tile shared with neighbouring workgroups is finished
// by the last of them to arrive: each publishes its partial through the workspace with 16-byte
// device-coherent stores, waits for them, and takes a ticket from the tile's counter; the last
// one adds the partials in workgroup order (bitwise deterministic) and resets the counter.
//
// Pipeline: a 4-deep ring of register stages, one 64-K step each (the weight fragment of every
// matrix, the bfp8 exponent dword, the B fragments); every load is unconditional (steps past the
// end of a wave's range re-load its last step) so the compiler never waits for more than the
// stage it consumes.
#include <algorithm>

#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

struct StParams {
  const uint8_t* w0;
  const uint8_t* w1;
  const int* rowexp0;  // bfp8: true weight = dequantised * 2^rowexp[row]
  const int* rowexp1;
  const uint16_t* src;  // B rows [M, K] bf16: x for gate/up, h for down
  int M, K, N, C, T;
  int P;                // workgroups
  int S;                // 64-K steps = 4 * T * C
  int maxseg;           // tiles one wave may touch
  void* out;            // gate/up: h [M, N] bf16; down: out [M, N] bf16 or fp32
  const void* residual; // down: [M, N] bf16 or fp32, may alias out
  int out_f32, res_f32;
  float* part;          // [P][2][NMAT * MG * 64] f32x4: partials of the first / last tile
  int* counters;        // [T] arrival counters (left at zero)
};

template <int WF, int NMAT, int MG>
struct SStage {
  typename StepWord<WF>::type w[NMAT][WF ? 1 : 2];
  uint32_t e[NMAT];
  u32x4 b[MG][2];
};

// Device-coherent 16-byte partial exchange (the sc1 cache policy of agent-scope atomics on a
// whole 16-byte lane, so one instruction moves whole lines); the descriptor bounds every access.
constexpr int kCoherentPolicy = 16;
constexpr int kRawBufferWord3 = 0x00020000;
__device__ __forceinline__ void st_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), r, off, 0, kCoherentPolicy);
}
__device__ __forceinline__ f32x4 ld_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCoherentPolicy));
}

// WG containing step s: the largest w with floor(w * S / P) <= s.
__device__ __forceinline__ int wg_of_step(int s, int S, int P) { return (int)(((long)(s + 1) * P - 1) / S); }

template <int WF, int NMAT, int MG, int NW>
__global__ __launch_bounds__(NW * 64) void stream_kernel(StParams p) {
  constexpr int BLK = WF == 2 ? kBf4Block : (WF ? kBfp8Block : kBf16Block);
  constexpr int SB = WF ? 1024 : 2048;
  constexpr int NACC = NMAT * MG;      // accumulated tiles per wave
  constexpr int CH = NACC >= 4 ? 1 : 2;  // independent product chains per tile
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = xcd_logical(blockIdx.x, p.P);
  const int SPT = p.C * kSteps;
  const int s0 = (int)((long)w * p.S / p.P), s1 = (int)((long)(w + 1) * p.S / p.P);
  const int sa = s0 + (int)((long)wave * (s1 - s0) / NW), sb = s0 + (int)((long)(wave + 1) * (s1 - s0) / NW);
  const int n = sb - sa;
  f32x4* slots = (f32x4*)lds;  // [NW][maxseg][NACC][64]

  // per-lane constant offsets
  const uint32_t lw = (uint32_t)lane * 16u, le = (WF == 2 ? 2048u : 4096u) + (uint32_t)lane * 4u;
  uint32_t boff[MG];  // byte offset of this lane's B row and quarter
#pragma unroll
  for (int g = 0; g < MG; ++g) {
    const int m = min(g * 16 + (lane & 15), p.M - 1);  // rows beyond M repeat row M - 1
    boff[g] = (uint32_t)(m * p.K + (lane >> 4) * 16) * 2u;
  }
  const uint8_t* srcb = (const uint8_t*)p.src;

  // Load the stage of step st (clamped into the wave's range; a wave without steps loads s0).
  auto load = [&](SStage<WF, NMAT, MG>& stg, int st) {
    const int sc = n > 0 ? min(st, sb - 1) : s0;
    const int tile = sc / SPT, ks = sc - tile * SPT;
    const size_t blk = ((size_t)tile * p.C + (ks >> 2)) * BLK;
    const uint32_t wo = WF == 2 ? (uint32_t)(ks & 2) * 512u + (uint32_t)(ks & 1) * 8u : (uint32_t)(ks & 3) * SB;
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      const uint8_t* b = (mat ? p.w1 : p.w0) + blk;
      stg.w[mat][0] = ld_stream((const typename StepWord<WF>::type*)(b + wo + lw));
      if constexpr (WF) {
        stg.e[mat] = ld_stream((const uint32_t*)(b + le));
      } else {
        stg.w[mat][1] = ld_stream((const u32x4*)(b + wo + 1024 + lw));
      }
    }
    const uint8_t* bb = srcb + (size_t)ks * 128;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      stg.b[g][0] = *(const u32x4*)(bb + boff[g]);
      stg.b[g][1] = *(const u32x4*)(bb + boff[g] + 16);
    }
  };

  f32x4 acc[NACC][CH];
#pragma unroll
  for (int i = 0; i < NACC; ++i)
#pragma unroll
    for (int c = 0; c < CH; ++c) acc[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int tw0 = (n > 0 ? sa : s0) / SPT;  // first tile of this wave
  int cur = tw0;                             // tile being accumulated
  auto park = [&]() {
    f32x4* slot = slots + (size_t)((wave * p.maxseg + (cur - tw0)) * NACC) * 64 + lane;
#pragma unroll
    for (int i = 0; i < NACC; ++i) {
      slot[i * 64] = CH == 2 ? acc[i][0] + acc[i][CH - 1] : acc[i][0];
#pragma unroll
      for (int c = 0; c < CH; ++c) acc[i][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto compute = [&](const SStage<WF, NMAT, MG>& stg, int st) {
    const int tile = st / SPT;
    if (tile != cur) {
      park();
      cur = tile;
    }
    const int j = (st - tile * SPT) & 3;
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat) {
      bf16x8 a0, a1;
      if constexpr (WF == 2) {
        dq16_bf4_bf16(stg.w[mat][0].x, stg.w[mat][0].y, (stg.e[mat] >> (8 * j)) & 0xffu, a0, a1);
      } else if constexpr (WF) {
        dq16_bf16(stg.w[mat][0], (stg.e[mat] >> (8 * j)) & 0xffu, a0, a1);
      } else {
        a0 = __builtin_bit_cast(bf16x8, stg.w[mat][0]);
        a1 = __builtin_bit_cast(bf16x8, stg.w[mat][1]);
      }
#pragma unroll
      for (int g = 0; g < MG; ++g) {
        const int i = mat * MG + g;
        acc[i][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, __builtin_bit_cast(bf16x8, stg.b[g][0]), acc[i][0], 0, 0, 0);
        acc[i][CH - 1] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, __builtin_bit_cast(bf16x8, stg.b[g][1]), acc[i][CH - 1], 0, 0, 0);
      }
    }
  };

  SStage<WF, NMAT, MG> q0, q1, q2, q3;
  // The scheduling fences keep each load after the compute that frees its stage: hoisting the
  // loads would make the compiler rename (copy) whole stages and wait for them.
  auto step = [&](SStage<WF, NMAT, MG>& stg, int st, int next) {
    compute(stg, st);
    __builtin_amdgcn_sched_barrier(0);
    load(stg, next);
    __builtin_amdgcn_sched_barrier(0);
  };
  load(q0, sa);
  load(q1, sa + 1);
  load(q2, sa + 2);
  load(q3, sa + 3);
  const int nit = n >= 8 ? (n - 4) / 4 : 0;  // iterations whose four loads all stay in range
  for (int it = 0; it < nit; ++it) {
    const int b = sa + 4 * it;
    step(q0, b, b + 4);
    step(q1, b + 1, b + 5);
    step(q2, b + 2, b + 6);
    step(q3, b + 3, b + 7);
  }
  // tail: r = n - i <= 7 steps left, steps i..i+3 are loaded; the loads of later steps are
  // issued unconditionally (clamped duplicates past the end)
  const int i = 4 * nit;
  const int r = n - i;
  if (r > 0) compute(q0, sa + i);
  __builtin_amdgcn_sched_barrier(0);
  load(q0, sa + i + 4);
  __builtin_amdgcn_sched_barrier(0);
  if (r > 1) compute(q1, sa + i + 1);
  __builtin_amdgcn_sched_barrier(0);
  load(q1, sa + i + 5);
  __builtin_amdgcn_sched_barrier(0);
  if (r > 2) compute(q2, sa + i + 2);
  __builtin_amdgcn_sched_barrier(0);
  load(q2, sa + i + 6);
  __builtin_amdgcn_sched_barrier(0);
  if (r > 3) compute(q3, sa + i + 3);
  if (r > 4) compute(q0, sa + i + 4);
  if (r > 5) compute(q1, sa + i + 5);
  if (r > 6) compute(q2, sa + i + 6);
  if (n > 0) park();
  __syncthreads();

  // ---- finish: the tiles of this workgroup, one wave per tile
  const int tfirst = s0 / SPT, tlast = (s1 - 1) / SPT;
  const __amdgpu_buffer_rsrc_t prs =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.part, 0, p.P * 2 * NACC * 64 * 16, kRawBufferWord3);
  for (int t = tfirst + wave; t <= tlast; t += NW) {
    f32x4 tot[NACC];
#pragma unroll
    for (int k = 0; k < NACC; ++k) tot[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int v = 0; v < NW; ++v) {
      const int va = s0 + (int)((long)v * (s1 - s0) / NW), vb = s0 + (int)((long)(v + 1) * (s1 - s0) / NW);
      if (va >= vb) continue;
      const int v0 = va / SPT, v1 = (vb - 1) / SPT;
      if (t < v0 || t > v1) continue;
      const f32x4* slot = slots + (size_t)((v * p.maxseg + (t - v0)) * NACC) * 64 + lane;
#pragma unroll
      for (int k = 0; k < NACC; ++k) tot[k] += slot[k * 64];
    }
    const int ta = t * SPT, tb = ta + SPT;  // the tile's steps
    if (ta < s0 || tb > s1) {
      // shared with neighbouring workgroups: publish, arrive, the last one finishes
      const int wa = wg_of_step(ta, p.S, p.P), wb = wg_of_step(tb - 1, p.S, p.P);
      const uint32_t mine = (uint32_t)((w * 2 + (t == tfirst ? 0 : 1)) * NACC * 64 + lane) * 16u;
#pragma unroll
      for (int k = 0; k < NACC; ++k) st_coherent(prs, mine + k * 1024u, tot[k]);
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);  // the partial has reached memory
      int last = 0;
      if (lane == 0) {
        const int old = __hip_atomic_fetch_add(p.counters + t, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == wb - wa;
        if (last) __hip_atomic_store(p.counters + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      last = __builtin_amdgcn_readfirstlane(last);
      if (!last) continue;
      // sum every workgroup's partial in workgroup order (this one's from registers)
      f32x4 sum[NACC];
#pragma unroll
      for (int k = 0; k < NACC; ++k) sum[k] = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int u = wa; u <= wb; ++u) {
        if (u == w) {
#pragma unroll
          for (int k = 0; k < NACC; ++k) sum[k] += tot[k];
          continue;
        }
        const int ut0 = (int)((long)u * p.S / p.P) / SPT;  // first tile of workgroup u
        const uint32_t off = (uint32_t)((u * 2 + (t == ut0 ? 0 : 1)) * NACC * 64 + lane) * 16u;
        f32x4 v[NACC];
#pragma unroll
        for (int k = 0; k < NACC; ++k) v[k] = ld_coherent(prs, off + k * 1024u);
#pragma unroll
        for (int k = 0; k < NACC; ++k) sum[k] += v[k];
      }
#pragma unroll
      for (int k = 0; k < NACC; ++k) tot[k] = sum[k];
    }
    // epilogue: lane l holds rows 4 * (l / 16) + (0..3) of tile t for token g * 16 + l % 16
    const int nb = t * kTileRows + (lane >> 4) * 4;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      const int m = g * 16 + (lane & 15);
      if (m >= p.M) continue;
      if constexpr (NMAT == 2) {
        uint16_t o[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float gv = tot[g][v], uv = tot[MG + g][v];
          if constexpr (WF) {
            gv = __builtin_amdgcn_ldexpf(gv, p.rowexp0[nb + v]);
            uv = __builtin_amdgcn_ldexpf(uv, p.rowexp1[nb + v]);
          }
          o[v] = f32_to_bf16(silu_mul(gv, uv));
        }
        *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + nb) =
            u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      } else {
        float y[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          y[v] = tot[g][v];
          if constexpr (WF) y[v] = __builtin_amdgcn_ldexpf(y[v], p.rowexp0[nb + v]);
        }
        if (p.residual) {
          if (p.res_f32) {
            const f32x4 rr = *(const f32x4*)((const float*)p.residual + (size_t)m * p.N + nb);
#pragma unroll
            for (int v = 0; v < 4; ++v) y[v] += rr[v];
          } else {
            const u32x2 rr = *(const u32x2*)((const uint16_t*)p.residual + (size_t)m * p.N + nb);
            y[0] += bf16_to_f32((uint16_t)(rr.x & 0xffffu));
            y[1] += bf16_to_f32((uint16_t)(rr.x >> 16));
            y[2] += bf16_to_f32((uint16_t)(rr.y & 0xffffu));
            y[3] += bf16_to_f32((uint16_t)(rr.y >> 16));
          }
        }
        if (p.out_f32) {
          *(f32x4*)((float*)p.out + (size_t)m * p.N + nb) = f32x4{y[0], y[1], y[2], y[3]};
        } else {
          *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + nb) =
              u32x2{(uint32_t)f32_to_bf16(y[0]) | ((uint32_t)f32_to_bf16(y[1]) << 16),
                    (uint32_t)f32_to_bf16(y[2]) | ((uint32_t)f32_to_bf16(y[3]) << 16)};
        }
      }
    }
  }
}

// ---------------------------------------------------------------- host side

constexpr int kStNW = 8;
constexpr int kStMaxSeg = 4;

// Workgroups for one projection: one per CU, fewer when there are fewer steps than that, more
// when a wave's range would cross more than kStMaxSeg tiles.
int plan_stream(int rows, int K, int num_cus, int* P_out, int* maxseg_out) {
  if (rows <= 0 || K <= 0 || rows % kTileRows || K % kSuperK) return -1;
  const long T = rows / kTileRows, SPT = (long)(K / kSuperK) * kSteps, S = T * SPT;
  int P = std::max(1, std::min(num_cus < 1 ? 1 : num_cus, kMaxWorkgroups));
  if (P > S) P = (int)S;
  for (;;) {
    const long per_wave = (S + (long)P * kStNW - 1) / ((long)P * kStNW) + 1;
    const int maxseg = (int)((per_wave - 1 + SPT - 1) / SPT) + 1;
    if (maxseg <= kStMaxSeg || P >= kMaxWorkgroups || P >= S) {
      if (maxseg > kStMaxSeg) return -2;
      *P_out = P;
      *maxseg_out = maxseg;
      return 0;
    }
    P = std::min<long>(std::min<long>(kMaxWorkgroups, S), P * 2);
  }
}

bool stream_supported(int M, int H, int I, int num_cus) {
  int P, ms;
  return M >= 1 && M <= 32 && plan_stream(I, H, num_cus, &P, &ms) == 0 && plan_stream(H, I, num_cus, &P, &ms) == 0;
}

template <int WF, int NMAT, int MG>
static int launch_stream(const StParams& p, hipStream_t s) {
  const size_t lds = (size_t)kStNW * p.maxseg * NMAT * MG * 64 * 16;
  launch_timed(NMAT == 2 ? 0 : 1, stream_kernel<WF, NMAT, MG, kStNW>, dim3(p.P), dim3(kStNW * 64), lds, s, p);
  return check_launch("stream_kernel");
}

template <int WF, int NMAT>
static int launch_stream_m(const StParams& p, hipStream_t s) {
  return p.M <= 16 ? launch_stream<WF, NMAT, 1>(p, s) : launch_stream<WF, NMAT, 2>(p, s);
}

int launch_forward_stream(const ForwardArgs& a, int num_cus, hipStream_t s) {
  const WsLayout L = ws_layout(a.M, a.H, a.I, a.fmt);
  const int fmt = a.fmt;
  int Pg, mg, Pd, md;
  if (plan_stream(a.I, a.H, num_cus, &Pg, &mg) || plan_stream(a.H, a.I, num_cus, &Pd, &md))
    return set_error(-1, "no weight-streaming split for H=%d I=%d", a.H, a.I);
  uint16_t* h = (uint16_t*)(a.ws + L.h);
  StParams g{};
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
  g.P = Pg;
  g.S = g.T * g.C * kSteps;
  g.maxseg = mg;
  g.out = h;
  g.part = (float*)(a.ws + L.part_gu);
  g.counters = (int*)(a.ws + L.counters_gu);
  int rc = fmt == 2 ? launch_stream_m<2, 2>(g, s) : (fmt == 1 ? launch_stream_m<1, 2>(g, s) : launch_stream_m<0, 2>(g, s));
  if (rc) return rc;
  StParams d{};
  d.w0 = a.wd;
  const int dfmt = down_format(fmt);
  d.rowexp0 = (const int*)(a.wd + rowexp_offset(a.H, a.I, dfmt));
  d.src = h;
  d.M = a.M;
  d.K = a.I;
  d.N = a.H;
  d.C = a.I / kSuperK;
  d.T = a.H / kTileRows;
  d.P = Pd;
  d.S = d.T * d.C * kSteps;
  d.maxseg = md;
  d.out = a.out;
  d.residual = a.residual;
  d.out_f32 = a.out_f32;
  d.res_f32 = a.res_f32;
  d.part = (float*)(a.ws + L.part_d);
  d.counters = (int*)(a.ws + L.counters_d);
  rc = dfmt == 1 ? launch_stream_m<1, 1>(d, s) : launch_stream_m<0, 1>(d, s);
  if (rc) return rc;
  return 0;
}

}  // namespace qmlp
