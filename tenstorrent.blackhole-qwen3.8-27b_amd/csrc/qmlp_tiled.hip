// qmlp_tiled.hip -- matrix-core GEMM kernels for many tokens (prefill chunks).
//
// Reference realisation being replaced: the prefill branch of Qwen36MLP -- the fused gate/up
// with SiLU on fp32 accumulators (docker/qwen-c2-graft/graft/mlp.py:440-456, rounded once,
// docs/real-text-2026-09-24.md:272-276) and the down projection with its prefill program config
// (mlp.py:539-611).
//
// Formulation: out^T[n, m] = sum_k W[n, k] x[m, k].  The weights are the matrix-core A operand:
// each wave owns TPW 16-row tiles of each matrix and streams them through registers in the packed
// layout (bfp8 and bf4 dequantised exactly to fp16 in registers, bf16 used as is).  The tokens are the
// B operand: a block stages MG groups of 16 token rows, one 64-K step at a time, into a 3-slot LDS
// ring shared by all its waves (bfrag_off's order, the same as the weight-streaming kernels', so
// each lane reads its B fragment with two 16-byte LDS loads).  One block = NWV waves x TPW tiles x
// NMAT matrices of features by MG x 16 tokens; every A fragment feeds MG x 2 products and every B
// fragment NMAT x TPW x 2.
//
// Pipeline per 64-K step s: compute step s from LDS slot s%3 and register stage s%3; issue the
// weight loads of step s+3 into that stage; write the B rows of step s+2 (requested one or three
// steps earlier, by the number of B register buffers) into slot (s+2)%3; one barrier.  The row
// exponents of a 256-K superblock (one 32-bit word per lane and tile) are requested once per
// superblock, a superblock ahead.  Loads beyond the last step are clamped duplicates, so every
// weight and B load is unconditional.
//
// Epilogue (fp32 accumulators in registers): gate/up -> h = silu(g) * u rounded once (fp16 *
// 2^th for bfp8, bf16 for bf16 weights); down -> out = residual + y.  Every output element is
// owned by one lane of one wave, except in the tiles that follow the last whole round of resident
// blocks: those split their K range over a few blocks, whose fp32 partial tiles meet in the
// workspace and are added in a fixed order (deterministic), each token group by one block.
#include <map>
#include <mutex>
#include <type_traits>

#include "qmlp_common.h"
#include "qmlp_internal.h"

namespace qmlp {

struct TlParams {
  const uint8_t* w0;
  const uint8_t* w1;
  const int* rowexp0;
  const int* rowexp1;
  const uint16_t* src;   // [M, K] B rows: fp16 * 2^tsrc[m] (bfp8 weights) or bf16
  int M, K, N, C;        // N output features, C = K / 256
  int nbm;               // token blocks
  int bn0;               // first feature block of the K-split part
  int ks;                // down projection: K splits per tile of the K-split part (1: no split)
  int nfull;             // leading blocks that cover whole K ranges of feature blocks 0, 1, ...
                         // (tiled_kernel; the K-split part follows them in the same launch)
  int ntail;             // tiled32_kernel: split tiles (blocks of padding tiles beyond exit)
  float* part;           // ks > 1: fp32 partial tiles, [tile][K split][block's outputs]
  int part_bytes;
  int* counters;         // ks > 1: arrival counter per tile (tiled_kernel), publication counter
                         // per split tile (tiled32_kernel); left at zero
  const int* tsrc;       // bfp8: per-token exponent of src
  const int* tout;       // bfp8 gate/up: h16 = h * 2^tout[m]
  void* out;             // gate/up: h [M, N] 16-bit; down: out [M, N] bf16 or fp32
  const void* residual;  // down: [M, N] bf16 or fp32, may alias out
  int out_f32, res_f32;
};

// Runs steps s .. nst-1 of a block's K loop, unrolled by U (the period of the register stage and
// buffer rotation): step(k, s) runs step s, k = s % U (a constant of each unrolled copy).
template <int U, typename F>
__device__ __forceinline__ void run_steps(int s, int nst, F&& step) {
  for (; s + U <= nst; s += U)
#pragma unroll
    for (int k = 0; k < U; ++k) step(k, s + k);
  const int r = nst - s;
#pragma unroll
  for (int k = 0; k < U - 1; ++k)
    if (k < r) step(k, s + k);
}

template <int WF, int NMAT, int TPW>
struct TlStage {
  typename StepWord<WF>::type w[NMAT][TPW][WF ? 1 : 2];
};

template <int WF, int NMAT, int TPW, int MG, int NWV, int NBB>
__global__ __launch_bounds__(NWV * 64) void tiled_kernel(TlParams p) {
  constexpr int NT = NWV * 64;
  constexpr int SLOT = MG * 2048;      // LDS bytes of one 64-K step of B
  // 16-byte B chunks per loading thread per step; with fewer chunks than threads (one group of
  // tokens) only the first NLD threads (whole waves) load
  constexpr int CPT = (MG * 128 + NT - 1) / NT, NLD = MG * 128 / CPT;
  static_assert(CPT * NLD == MG * 128 && NLD <= NT && NLD % 64 == 0, "B chunks must divide evenly over whole waves");
  constexpr int BLK = WF == 2 ? kBf4Block : (WF ? kBfp8Block : kBf16Block);
  constexpr int SB = WF ? 1024 : 2048;  // bytes of one bf16/bfp8 K-step inside a weight block
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // A launch holds up to two parts: blocks [0, nfull) each cover the whole K range of one tile
  // of feature blocks 0, 1, ...; the rest split the K range of each tile of feature blocks
  // bn0, ... into ks parts.  The hardware dispatches blocks in index order as earlier ones
  // retire, so the short K-split blocks fill the CUs that finish their whole-K blocks first
  // (on a CU the block dispatched first finishes ~25 % sooner than the second).
  const bool full = (int)blockIdx.x < p.nfull;
  const int b = full ? (int)blockIdx.x : (int)blockIdx.x - p.nfull;
  const int L = xcd_logical(b, full ? p.nfull : (int)gridDim.x - p.nfull);  // blocks sharing weights share an XCD
  const int ks = full ? 1 : p.ks;
  // tile = (feature block, token block); with K splits, the ks blocks of a tile are consecutive
  const int tile = L / ks, q = L % ks;
  const int bn = (full ? 0 : p.bn0) + tile / p.nbm, bm = tile % p.nbm;
  const int m0 = bm * MG * 16;
  const int tile0 = (bn * NWV + wave) * TPW;
  // K range of this block: superblocks [q C / ks, (q + 1) C / ks), steps counted from kbase
  const int kbase = q * p.C / ks * kSteps;
  const int nst = (q + 1) * p.C / ks * kSteps - kbase;

  // B chunk c = threadIdx.x + i * NT: token row r = c / 8, 8 K values j = c % 8 of the step;
  // quarter j / 2, half j % 2.  Rows beyond M repeat row M - 1 (their outputs are not stored).
  // Every load goes through a buffer descriptor whose base is uniform (the block's token rows,
  // the wave's weight tiles): the lane's byte offset is a constant 32-bit register and the
  // step's offset a uniform scalar, so no load needs per-lane 64-bit address arithmetic.
  const int brows = min(MG * 16, p.M - m0);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.src + (size_t)m0 * p.K * 2), 0, brows * p.K * 2, kBufferRsrcWord3);
  uint32_t goff[CPT], loff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = min((int)threadIdx.x, NLD - 1) + i * NLD, r = c >> 3, j = c & 7;
    const int mr = min(r, brows - 1);
    goff[i] = (uint32_t)(mr * p.K + j * 8) * 2u;
    loff[i] = (uint32_t)(r >> 4) * 2048u + bfrag_off(j >> 1, r & 15, j & 1);
  }
  const bool loader = NLD == NT || (int)threadIdx.x < NLD;  // whole waves
  auto bload = [&](u32x4(&v)[CPT], int step) {
    const int so = (kbase + min(step, nst - 1)) * 128;
    if (loader)
#pragma unroll
      for (int i = 0; i < CPT; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, goff[i], so, 0);
  };
  auto bstore = [&](const u32x4(&v)[CPT], int step) {
    uint8_t* slot = lds + (step % 3) * SLOT;
    if (loader)
#pragma unroll
      for (int i = 0; i < CPT; ++i) *(u32x4*)(slot + loff[i]) = v[i];
  };

  const int tile_bytes = p.C * BLK;
  __amdgpu_buffer_rsrc_t wr[NMAT];  // the wave's TPW tiles of each matrix
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
    wr[mat] = __builtin_amdgcn_make_buffer_rsrc((void*)((mat ? p.w1 : p.w0) + (size_t)tile0 * tile_bytes), 0,
                                                TPW * tile_bytes, kBufferRsrcWord3);
  const uint32_t lw = (uint32_t)lane * 16u, le = (WF == 2 ? 2048u : 4096u) + (uint32_t)lane * 4u;
  // Weights are re-read by every token block of the same features, so they are loaded with the
  // default cache policy (kept in L2 for the neighbouring blocks of the XCD).
  auto wload = [&](TlStage<WF, NMAT, TPW>& st, int step) {
    const int sc = kbase + min(step, nst - 1);  // kbase is a multiple of 4: sc & 3 == step & 3
    const int so = (sc >> 2) * BLK + (WF == 2 ? (sc & 2) * 512 + (sc & 1) * 8 : (sc & 3) * SB);
#pragma unroll
    for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const uint32_t vo = (uint32_t)(t * tile_bytes) + lw;
        if constexpr (WF == 2) {
          st.w[mat][t][0] = __builtin_amdgcn_raw_buffer_load_b64(wr[mat], vo, so, 0);
        } else {
          st.w[mat][t][0] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], vo, so, 0);
          if constexpr (!WF) st.w[mat][t][1] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], vo + 1024u, so, 0);
        }
      }
  };
  // Row exponents: the lane's 32-bit word of a tile's superblock holds the group exponents of
  // the superblock's 4 K-steps (byte j: step j), so it is requested once per superblock, one
  // superblock ahead of its use (ecur: the superblock being computed, enext: the next one).
  // Requested with every step's weights, it made 2 of the 5 vector memory instructions of a
  // down-projection step, on kernels bound by their vector memory path.
  uint32_t ecur[NMAT][TPW], enext[NMAT][TPW];
  const int nsb = nst / kSteps;
  auto eload = [&](uint32_t(&e)[NMAT][TPW], int sb) {
    if constexpr (WF != 0) {
      const int so = (kbase / kSteps + min(sb, nsb - 1)) * BLK;
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int t = 0; t < TPW; ++t)
          e[mat][t] = __builtin_amdgcn_raw_buffer_load_b32(wr[mat], (uint32_t)(t * tile_bytes) + le, so, 0);
    }
  };
  auto erotate = [&](int sb) {  // after the last step of superblock sb
    if constexpr (WF != 0) {
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int t = 0; t < TPW; ++t) ecur[mat][t] = enext[mat][t];
      eload(enext, sb + 2);
    }
  };

  f32x4 acc[NMAT][TPW][MG];
#pragma unroll
  for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
    for (int t = 0; t < TPW; ++t)
#pragma unroll
      for (int g = 0; g < MG; ++g) acc[mat][t][g] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t boff0 = bfrag_off(lane >> 4, lane & 15, 0), boff1 = bfrag_off(lane >> 4, lane & 15, 1);
  // kq = step % 4: the step's byte of the exponent word
  auto compute = [&](const TlStage<WF, NMAT, TPW>& st, int step, int kq) {
    const uint8_t* slot = lds + (step % 3) * SLOT;
    if constexpr (WF) {
      f16x8 a[NMAT][TPW][2];
#pragma unroll
      for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
          if constexpr (WF == 2)
            dq16_bf4(st.w[mat][t][0].x, st.w[mat][t][0].y, scale_pair(ecur[mat][t], kq), a[mat][t][0],
                     a[mat][t][1]);
          else
            dq16(st.w[mat][t][0], scale_pair(ecur[mat][t], kq), a[mat][t][0], a[mat][t][1]);
        }
#pragma unroll
      for (int g = 0; g < MG; ++g) {
        const f16x8 b0 = __builtin_bit_cast(f16x8, *(const u32x4*)(slot + g * 2048 + boff0));
        const f16x8 b1 = __builtin_bit_cast(f16x8, *(const u32x4*)(slot + g * 2048 + boff1));
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int t = 0; t < TPW; ++t) {
            acc[mat][t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mat][t][0], b0, acc[mat][t][g], 0, 0, 0);
            acc[mat][t][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[mat][t][1], b1, acc[mat][t][g], 0, 0, 0);
          }
      }
    } else {
#pragma unroll
      for (int g = 0; g < MG; ++g) {
        const bf16x8 b0 = __builtin_bit_cast(bf16x8, *(const u32x4*)(slot + g * 2048 + boff0));
        const bf16x8 b1 = __builtin_bit_cast(bf16x8, *(const u32x4*)(slot + g * 2048 + boff1));
#pragma unroll
        for (int mat = 0; mat < NMAT; ++mat)
#pragma unroll
          for (int t = 0; t < TPW; ++t) {
            acc[mat][t][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.w[mat][t][0]), b0,
                                                                     acc[mat][t][g], 0, 0, 0);
            acc[mat][t][g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, st.w[mat][t][1]), b1,
                                                                     acc[mat][t][g], 0, 0, 0);
          }
      }
    }
  };

  // B rows travel global -> registers -> LDS.  NBB = 3 register buffers give every B load three
  // iterations to land (step s+5 is requested in iteration s, like the weight stages); NBB = 2
  // gives one (step s+3 is requested at the top of iteration s) for the kernels whose occupancy
  // the third buffer's registers would halve.
  constexpr int U = NBB == 3 ? 3 : 6;
  TlStage<WF, NMAT, TPW> s0, s1, s2;
  u32x4 b0[CPT], b1[CPT], b2[CPT];
  bload(b0, 0);
  bload(b1, 1);
  eload(ecur, 0);
  wload(s0, 0);
  wload(s1, 1);
  wload(s2, 2);
  eload(enext, 1);
  bstore(b0, 0);
  bstore(b1, 1);
  bload(b2, 2);
  int s = 0;
  // iteration k of the unroll: stage k % 3 computes step s and then receives step s+3; after a
  // superblock's last step (a uniform branch) the exponent words move on
  auto stage = [&](int i) -> TlStage<WF, NMAT, TPW>& { return i == 0 ? s0 : (i == 1 ? s1 : s2); };
  if constexpr (NBB == 3) {
    bload(b0, 3);
    bload(b1, 4);
    __syncthreads();
    // iteration s: the buffer holding step s+2 goes to LDS slot (s+2) % 3 (last read in
    // iteration s-1) and then receives step s+5.
    run_steps<U>(s, nst, [&](int k, int s) {
      TlStage<WF, NMAT, TPW>& cur = stage(k % 3);
      u32x4(&bw)[CPT] = k % 3 == 0 ? b2 : (k % 3 == 1 ? b0 : b1);
      compute(cur, s, s & 3);
      wload(cur, s + 3);
      bstore(bw, s + 2);
      bload(bw, s + 5);
      if ((s & 3) == 3) erotate(s / kSteps);
      __syncthreads();
    });
  } else {
    __syncthreads();
    // iteration s: bnext receives step s+3 (it held step s+1, already in LDS); bwrite holds step
    // s+2 and goes to slot (s+2) % 3, which was last read in iteration s-1.
    run_steps<U>(s, nst, [&](int k, int s) {
      TlStage<WF, NMAT, TPW>& cur = stage(k % 3);
      u32x4(&bnext)[CPT] = k % 2 == 0 ? b1 : b2;
      u32x4(&bwrite)[CPT] = k % 2 == 0 ? b2 : b1;
      bload(bnext, s + 3);
      compute(cur, s, s & 3);
      wload(cur, s + 3);
      bstore(bwrite, s + 2);
      if ((s & 3) == 3) erotate(s / kSteps);
      __syncthreads();
    });
  }

  if constexpr (NMAT == 1) {
    if (ks > 1) {
      // K-split tail: publish the partial tile, arrive; the last of the tile's ks blocks adds
      // the ks partials in K order (deterministic) and runs the epilogue.
      __shared__ int s_last;
      const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(p.part, 0, p.part_bytes, kBufferRsrcWord3);
      auto slot = [&](int qq, int t, int g) {  // byte offset of this lane's f32x4 in split qq's tile
        return (uint32_t)(((((size_t)tile * ks + qq) * NWV + wave) * TPW * MG + t * MG + g) * 64 + lane) * 16u;
      };
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int g = 0; g < MG; ++g) store_coherent(prs, slot(q, t, g), acc[0][t][g]);
      wait_stores();
      __syncthreads();
      if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(p.counters + tile, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = old == ks - 1;
        if (s_last) __hip_atomic_store(p.counters + tile, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (!s_last) return;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int g = 0; g < MG; ++g) {
          f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
          for (int qq = 0; qq < ks; ++qq) sum += qq == q ? acc[0][t][g] : load_coherent(prs, slot(qq, t, g));
          acc[0][t][g] = sum;
        }
    }
  }

  // epilogue: lane l holds features 4 * (l / 16) + v of each tile for token l % 16 of each group
  const int col = lane & 15, rq = (lane >> 4) * 4;
#pragma unroll
  for (int g = 0; g < MG; ++g) {
    const int m = m0 + g * 16 + col;
    if (m >= p.M) continue;
    const int ts = WF ? p.tsrc[m] : 0;
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int n = (tile0 + t) * kTileRows + rq;
      uint16_t o[4];
      if constexpr (NMAT == 2) {
        const int to = WF ? p.tout[m] : 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float gv = acc[0][t][g][v], uv = acc[1][t][g][v];
          if constexpr (WF) {
            gv = __builtin_amdgcn_ldexpf(gv, p.rowexp0[n + v] - ts);
            uv = __builtin_amdgcn_ldexpf(uv, p.rowexp1[n + v] - ts);
          }
          const float hv = silu_mul(gv, uv);
          o[v] = WF ? f32_to_f16_bits(__builtin_amdgcn_ldexpf(hv, to)) : f32_to_bf16(hv);
        }
      } else {
        float y[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          y[v] = acc[0][t][g][v];
          if constexpr (WF) y[v] = __builtin_amdgcn_ldexpf(y[v], p.rowexp0[n + v] - ts);
        }
        if (p.residual) {
          if (p.res_f32) {
            const f32x4 rr = *(const f32x4*)((const float*)p.residual + (size_t)m * p.N + n);
#pragma unroll
            for (int v = 0; v < 4; ++v) y[v] += rr[v];
          } else {
            const u32x2 rr = *(const u32x2*)((const uint16_t*)p.residual + (size_t)m * p.N + n);
            y[0] += bf16_to_f32((uint16_t)(rr.x & 0xffffu));
            y[1] += bf16_to_f32((uint16_t)(rr.x >> 16));
            y[2] += bf16_to_f32((uint16_t)(rr.y & 0xffffu));
            y[3] += bf16_to_f32((uint16_t)(rr.y >> 16));
          }
        }
        if (p.out_f32) {
          *(f32x4*)((float*)p.out + (size_t)m * p.N + n) = f32x4{y[0], y[1], y[2], y[3]};
          continue;
        }
#pragma unroll
        for (int v = 0; v < 4; ++v) o[v] = f32_to_bf16(y[v]);
      }
      *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + n) =
          u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
    }
  }
}

// ---------------------------------------------------------------- 32 x 32 gate/up variant
//
// Dispatched for the block-float formats; the bf16 branch is kept so that the variant stays
// comparable across formats.
//
// Same formulation and pipeline as tiled_kernel (gate/up only), on 32x32x16 matrix-core products:
// each wave owns the 32-row feature pair (tiles 2 P and 2 P + 1) of both matrices for MG groups of
// 32 tokens.  Every 1 KB B fragment read from LDS then feeds two 32x32 products (65536 flops)
// instead of two 16x16 ones, and the wave issues half the matrix-core instructions, while every
// dequantised weight value still feeds MG x 32 tokens.
//
// A operand from the packed layout as it stands: lane l = 32 hk + 16 ts + r takes row r of tile
// 2 P + ts and the packed chunks q = 2 hk and 2 hk + 1 of each K-step (K = 64 j + 32 hk + 0..31),
// i.e. the 16-byte slots of packed lanes 32 hk + r and 32 hk + 16 + r.  Product u (0..3) of the
// step takes the lane's values 8 u .. 8 u + 7 of those 32: K = 64 j + 32 hk + 8 u + (0..7) on the
// lanes whose A index half is hk.  The B fragment of product u therefore holds, in lane
// l = 32 hk + c, the K values 64 j + 32 hk + 8 u + (0..7) of token c of the group.
typedef float f32x16 __attribute__((ext_vector_type(16)));

// 16-byte LDS slot of product u's B fragment for lane l inside one group's 4 KB step image.  The
// 8 lanes 8a..8a+7 of a fragment read one aligned 128-byte run (a rotation of it), and the 8 slots
// one token row writes per step (all (u, hk) pairs) fall on distinct 16-byte bank groups.
__host__ __device__ inline uint32_t b32_slot(int u, int l) {
  return (uint32_t)(u * 64 + (l & ~7) + ((l + 2 * u + (l >> 5)) & 7));
}

template <int WF, int NM>
struct Tl32Stage {
  typename StepWord<WF>::type w[NM][WF ? 2 : 4];
};

// K pieces per split tile of tiled32_kernel: 4 for the gate/up pair, 8 for the down projection
// (the last sums request every piece's chunks of a token group at once)
constexpr int kSplitMaxPieces = 8;

// NM = 2: gate/up (the wave's 32-row feature pair of both matrices); NM = 1: the down projection
// (one 32-row unit of its matrix per wave, residual epilogue).
//
// Work: blocks [0, nfull) each take one whole tile (tile = the block's logical index, feature
// blocks from bn0); blocks from nfull take K pieces of the ntail tiles that follow (rounded up to
// whole XCDs where every tile splits: the padding blocks exit at once): ks consecutive blocks
// share a tile, piece q covering 64-K steps [q S / ks, (q + 1) S / ks) of its S.  The whole tiles
// come in complete rounds of resident blocks and the pieces start together as those rounds end,
// so the blocks reading one feature block's weights read the same K range at the same time (L2
// reuse).  A split tile's pieces meet through the workspace by last arrival: every piece
// publishes its partial tile and counts itself, and the last to count adds the ks partials in K
// order and runs the epilogue.  No block ever waits for another, so the kernel cannot stall
// whatever else holds the CUs (other streams, other processes).
template <int WF, int MG, int NBB, int NM>
__global__ __launch_bounds__(512) void tiled32_kernel(TlParams p) {
  constexpr int NWV = 8, NT = NWV * 64;
  constexpr int SLOT = MG * 4096;     // LDS bytes of one 64-K step of B
  // 16-byte B chunks per loading thread per step (one group of tokens: the first NLD threads)
  constexpr int CPT = (MG * 256 + NT - 1) / NT, NLD = MG * 256 / CPT;
  static_assert(CPT * NLD == MG * 256 && NLD <= NT && NLD % 64 == 0, "B chunks must divide evenly over whole waves");
  constexpr int BLK = WF == 2 ? kBf4Block : (WF ? kBfp8Block : kBf16Block);
  constexpr uint32_t PART_BYTES = NWV * NM * MG * 16 * 64 * 4;  // one piece's partial tile
  extern __shared__ __align__(16) uint8_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool full = (int)blockIdx.x < p.nfull;
  const int b = full ? (int)blockIdx.x : (int)blockIdx.x - p.nfull;
  const int ks = full ? 1 : p.ks;
  // blocks sharing weights share an XCD (the pieces of a split tile too, where ks divides the
  // part's blocks per XCD: their partial tiles then meet in one L2)
  const int P = full ? p.nfull : (int)gridDim.x - p.nfull;
  const int L = full || (P / 8) % ks == 0 ? xcd_logical(b, P) : b;
  const int tt = L / ks, q = L % ks;  // split tiles: index among them, piece
  if (!full && tt >= p.ntail) return;  // a padding tile (the split tiles rounded up to whole XCDs)
  const int tile = full ? L : p.nfull + tt;
  const int bn = p.bn0 + tile / p.nbm, bm = tile % p.nbm;
  const int m0 = bm * MG * 32;
  const int pair = bn * NWV + wave;  // the wave's 32-row unit (of each matrix)
  // The piece's 64-K steps [kb, kb + nst) (every step of the K range for a whole tile; pieces cut
  // at step granularity, so that they differ by one step at most) and the superblocks they touch,
  // [k0, k0 + nsb); ph: the first step's position inside its superblock.
  const int kst = p.C * kSteps;
  const int kb = q * kst / ks, nst = (q + 1) * kst / ks - kb;
  const int k0 = kb / kSteps, nsb = (kb + nst - 1) / kSteps - k0 + 1, ph = kb % kSteps;
  // The epilogue's exponents (the block's NM x 256 row exponents, its 128 tokens' exponents)
  // staged in LDS after the B ring: requested first, written to LDS before the first barrier, read
  // after the last.  Kept out of the epilogue's global loads, which could not pass its stores.
  int* lexp = (int*)(lds + 3 * SLOT);  // [NM][NWV * 32] row exponents, then [2][MG * 32] token ones
  constexpr int NEXP = WF ? NM * NWV * 32 + (NM == 2 ? 2 : 1) * MG * 32 : 0;
  static_assert(NEXP <= 2 * NT, "two exponents per thread at most");
  int xval[2] = {0, 0};
  if constexpr (WF != 0) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int i = (int)threadIdx.x + r * NT;
      if (i < NM * NWV * 32) {
        const int* re = i < NWV * 32 ? p.rowexp0 : p.rowexp1;
        xval[r] = re[bn * NWV * 32 + (i & (NWV * 32 - 1))];
      } else if (i < NEXP) {
        const int j = i - NM * NWV * 32, mm = min(m0 + (j & (MG * 32 - 1)), p.M - 1);
        xval[r] = j < MG * 32 ? p.tsrc[mm] : p.tout[mm];
      }
    }
  }

  // B chunk c = threadIdx.x + i * NT: token row r = c / 8, K values 8 k8 .. 8 k8 + 7 of the step
  // (k8 = c % 8 = 4 hk + u).  Rows beyond M repeat row M - 1 (their outputs are not stored).
  // Every load goes through a buffer descriptor whose base is uniform (the block's token rows,
  // the wave's weight tiles): the lane's byte offset is a constant 32-bit register and the step's
  // offset a uniform scalar, so no load needs per-lane 64-bit address arithmetic.
  const int brows = min(MG * 32, p.M - m0);
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      (void*)((const uint8_t*)p.src + (size_t)m0 * p.K * 2), 0, brows * p.K * 2, kBufferRsrcWord3);
  uint32_t goff[CPT], loff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = min((int)threadIdx.x, NLD - 1) + i * NLD, r = c >> 3, k8 = c & 7;
    const int mr = min(r, brows - 1);
    goff[i] = (uint32_t)(mr * p.K + k8 * 8) * 2u;
    loff[i] = (uint32_t)(r >> 5) * 4096u + b32_slot(k8 & 3, 32 * (k8 >> 2) + (r & 31)) * 16u;
  }
  const bool loader = NLD == NT || (int)threadIdx.x < NLD;  // whole waves

  // Down projection: the residual words of the lane's outputs (group g, rows 8 vq + 0..3 of its
  // 4-row quarter), requested together after the K loop (by a split tile's last arrival, with
  // the other pieces' partials), so that they cost one round trip and none of the epilogue's
  // loads waits behind its stores.  Requested before the loop instead, their completion held up
  // the loop's first in-order waits (+5 us per block).  bf16: the low two words; fp32: all four.
  u32x4 rres[NM == 1 ? MG : 1][4];
#pragma unroll
  for (int g = 0; g < (NM == 1 ? MG : 1); ++g)
#pragma unroll
    for (int vq = 0; vq < 4; ++vq) rres[g][vq] = u32x4{0u, 0u, 0u, 0u};
  auto rload = [&]() {
    if constexpr (NM == 1) {
      if (!p.residual) return;
      const int col = lane & 31, rq = (lane >> 5) * 4;
#pragma unroll
      for (int g = 0; g < MG; ++g) {
        const size_t row = (size_t)min(m0 + g * 32 + col, p.M - 1) * p.N;
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int n = pair * 32 + vq * 8 + rq;
          if (p.res_f32) {
            rres[g][vq] = *(const u32x4*)((const float*)p.residual + row + n);
          } else {
            const u32x2 w = *(const u32x2*)((const uint16_t*)p.residual + row + n);
            rres[g][vq] = u32x4{w.x, w.y, 0u, 0u};
          }
        }
      }
    }
  };

  auto bload = [&](u32x4(&v)[CPT], int step) {
    const int so = (kb + min(step, nst - 1)) * 128;
    if (loader)
#pragma unroll
      for (int i = 0; i < CPT; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, goff[i], so, 0);
  };
  auto bstore = [&](const u32x4(&v)[CPT], int step) {
    uint8_t* slot = lds + (step % 3) * SLOT;
    if (loader)
#pragma unroll
      for (int i = 0; i < CPT; ++i) *(u32x4*)(slot + loff[i]) = v[i];
  };

  const int hk = lane >> 5;
  const int tile_bytes = p.C * BLK;
  __amdgpu_buffer_rsrc_t wr[NM];  // the wave's two 16-row tiles (2 pair, 2 pair + 1) of each matrix
#pragma unroll
  for (int mat = 0; mat < NM; ++mat)
    wr[mat] = __builtin_amdgcn_make_buffer_rsrc((void*)((mat ? p.w1 : p.w0) + (size_t)(2 * pair) * tile_bytes), 0,
                                                2 * tile_bytes, kBufferRsrcWord3);
  const uint32_t lp0 = (uint32_t)(32 * hk + (lane & 15)), lp1 = lp0 + 16u;
  const uint32_t wv = (uint32_t)((lane >> 4) & 1) * (uint32_t)tile_bytes;  // the lane's tile
  auto wload = [&](Tl32Stage<WF, NM>& st, int step) {
    const int sc = kb + min(step, nst - 1);
    const int bo = (sc >> 2) * BLK;
#pragma unroll
    for (int mat = 0; mat < NM; ++mat) {
      if constexpr (WF == 1) {
        const int so = bo + (sc & 3) * 1024;
        st.w[mat][0] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + lp0 * 16u, so, 0);
        st.w[mat][1] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + lp1 * 16u, so, 0);
      } else if constexpr (WF == 2) {
        const int so = bo + (sc & 2) * 512 + (sc & 1) * 8;
        st.w[mat][0] = __builtin_amdgcn_raw_buffer_load_b64(wr[mat], wv + lp0 * 16u, so, 0);
        st.w[mat][1] = __builtin_amdgcn_raw_buffer_load_b64(wr[mat], wv + lp1 * 16u, so, 0);
      } else {
        const int so = bo + (sc & 3) * 2048;
        st.w[mat][0] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + lp0 * 16u, so, 0);
        st.w[mat][1] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + 1024u + lp0 * 16u, so, 0);
        st.w[mat][2] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + lp1 * 16u, so, 0);
        st.w[mat][3] = __builtin_amdgcn_raw_buffer_load_b128(wr[mat], wv + 1024u + lp1 * 16u, so, 0);
      }
    }
  };

  // Row exponents, once per superblock and one superblock ahead, as in tiled_kernel: the lane's
  // words for its rows lp0 and lp1 of each matrix's tile.
  uint32_t ecur[NM][2], enext[NM][2];
  auto eload = [&](uint32_t(&e)[NM][2], int sb) {
    if constexpr (WF != 0) {
      const int so = (k0 + min(sb, nsb - 1)) * BLK + (WF == 2 ? 2048 : 4096);
#pragma unroll
      for (int mat = 0; mat < NM; ++mat) {
        e[mat][0] = __builtin_amdgcn_raw_buffer_load_b32(wr[mat], wv + lp0 * 4u, so, 0);
        e[mat][1] = __builtin_amdgcn_raw_buffer_load_b32(wr[mat], wv + lp1 * 4u, so, 0);
      }
    }
  };
  auto erotate = [&](int sb) {  // after the last step of the piece's superblock sb
    if constexpr (WF != 0) {
#pragma unroll
      for (int mat = 0; mat < NM; ++mat)
#pragma unroll
        for (int c = 0; c < 2; ++c) ecur[mat][c] = enext[mat][c];
      eload(enext, sb + 2);
    }
  };

  f32x16 acc[NM][MG];
#pragma unroll
  for (int mat = 0; mat < NM; ++mat)
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mat][g][v] = 0.f;

  uint32_t bs[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) bs[u] = b32_slot(u, lane) * 16u;
  // kq = step % 4: the step's byte of the exponent word
  auto compute = [&](const Tl32Stage<WF, NM>& st, int step, int kq) {
    const uint8_t* slot = lds + (step % 3) * SLOT;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      if constexpr (WF) {
        f16x8 a[NM][2];
#pragma unroll
        for (int mat = 0; mat < NM; ++mat) {
          if constexpr (WF == 2)
            dq16_bf4(st.w[mat][c].x, st.w[mat][c].y, scale_pair(ecur[mat][c], kq), a[mat][0], a[mat][1]);
          else
            dq16(st.w[mat][c], scale_pair(ecur[mat][c], kq), a[mat][0], a[mat][1]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int g = 0; g < MG; ++g) {
            const f16x8 b = __builtin_bit_cast(f16x8, *(const u32x4*)(slot + g * 4096 + bs[2 * c + h]));
#pragma unroll
            for (int mat = 0; mat < NM; ++mat)
              acc[mat][g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[mat][h], b, acc[mat][g], 0, 0, 0);
          }
      } else {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int g = 0; g < MG; ++g) {
            const bf16x8 b = __builtin_bit_cast(bf16x8, *(const u32x4*)(slot + g * 4096 + bs[2 * c + h]));
#pragma unroll
            for (int mat = 0; mat < NM; ++mat)
              acc[mat][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, st.w[mat][2 * c + h]),
                                                                    b, acc[mat][g], 0, 0, 0);
          }
      }
    }
  };

  // The pipeline of tiled_kernel: NBB = 3 B register buffers request step s+5 in iteration s,
  // NBB = 2 request step s+3 at the top of iteration s; weights of step s+3 are requested right
  // after step s's products; one barrier per step.
  constexpr int U = NBB == 3 ? 3 : 6;
  Tl32Stage<WF, NM> s0, s1, s2;
  u32x4 b0[CPT], b1[CPT], b2[CPT];
  bload(b0, 0);
  bload(b1, 1);
  eload(ecur, 0);
  wload(s0, 0);
  wload(s1, 1);
  wload(s2, 2);
  eload(enext, 1);
  bstore(b0, 0);
  bstore(b1, 1);
  bload(b2, 2);
  int s = 0;
  auto stage = [&](int i) -> Tl32Stage<WF, NM>& { return i == 0 ? s0 : (i == 1 ? s1 : s2); };
  if constexpr (WF != 0)
#pragma unroll
    for (int r = 0; r < 2; ++r)
      if ((int)threadIdx.x + r * NT < NEXP) lexp[threadIdx.x + r * NT] = xval[r];
  if constexpr (NBB == 3) {
    bload(b0, 3);
    bload(b1, 4);
    __syncthreads();
    run_steps<U>(s, nst, [&](int k, int s) {
      Tl32Stage<WF, NM>& cur = stage(k % 3);
      u32x4(&bw)[CPT] = k % 3 == 0 ? b2 : (k % 3 == 1 ? b0 : b1);
      compute(cur, s, (s + ph) & 3);
      wload(cur, s + 3);
      bstore(bw, s + 2);
      bload(bw, s + 5);
      if (((s + ph) & 3) == 3) erotate((s + ph) / kSteps);
      __syncthreads();
    });
  } else {
    __syncthreads();
    run_steps<U>(s, nst, [&](int k, int s) {
      Tl32Stage<WF, NM>& cur = stage(k % 3);
      u32x4(&bnext)[CPT] = k % 2 == 0 ? b1 : b2;
      u32x4(&bwrite)[CPT] = k % 2 == 0 ? b2 : b1;
      bload(bnext, s + 3);
      compute(cur, s, (s + ph) & 3);
      // keeps the next weight loads behind the products: hoisted above them, their registers
      // make the compiler wait for every LDS read before its two products
      __builtin_amdgcn_sched_barrier(0);
      wload(cur, s + 3);
      bstore(bwrite, s + 2);
      if (((s + ph) & 3) == 3) erotate((s + ph) / kSteps);
      __syncthreads();
    });
  }

  // Epilogue over the tile's outputs, one group of 32 tokens at a time: every value the group
  // needs (its accumulator chunks, partial tiles, residual words) is requested before any of its
  // stores, so each group costs one memory round trip.  chunk(mat, g, v4) gives accumulators
  // 4 v4 .. 4 v4 + 3 of matrix mat and group g.  Accumulator v of lane l holds row
  // 8 (v / 4) + 4 (l / 32) + v % 4 of the wave's 32-row unit for token l % 32 of the group.
  auto epilogue = [&](auto chunk) {
    const int col = lane & 31, rq = (lane >> 5) * 4;
    const int* lrow = lexp + wave * 32 + rq;    // this lane's rows: + 8 vq + v (+ NWV * 32 for up)
    const int* ltok = lexp + NM * NWV * 32 + col;  // this lane's token: + 32 g (+ MG * 32: tout)
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      const int m = m0 + g * 32 + col;
      const bool live = m < p.M;
      f32x4 a[NM][4];
#pragma unroll
      for (int mat = 0; mat < NM; ++mat)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) a[mat][vq] = chunk(mat, g, vq);
      const int ts = WF ? ltok[32 * g] : 0;
      if constexpr (NM == 1) {
        // down: out = residual + y, y = acc * 2^(row exponent - token exponent)
        if (!live) continue;
        f32x4 rr[4];
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const u32x4 w = rres[NM == 1 ? g : 0][vq];
          rr[vq] = p.res_f32 ? __builtin_bit_cast(f32x4, w)
                             : f32x4{bf16_to_f32((uint16_t)(w.x & 0xffffu)), bf16_to_f32((uint16_t)(w.x >> 16)),
                                     bf16_to_f32((uint16_t)(w.y & 0xffffu)), bf16_to_f32((uint16_t)(w.y >> 16))};
        }
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int n = pair * 32 + vq * 8 + rq;
          float y[4];
#pragma unroll
          for (int v = 0; v < 4; ++v)
            y[v] = (WF ? __builtin_amdgcn_ldexpf(a[0][vq][v], lrow[8 * vq + v] - ts) : a[0][vq][v]) + rr[vq][v];
          if (p.out_f32) {
            *(f32x4*)((float*)p.out + (size_t)m * p.N + n) = f32x4{y[0], y[1], y[2], y[3]};
          } else {
            const uint32_t o0 = f32_to_bf16(y[0]), o1 = f32_to_bf16(y[1]), o2 = f32_to_bf16(y[2]),
                           o3 = f32_to_bf16(y[3]);
            *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + n) = u32x2{o0 | (o1 << 16), o2 | (o3 << 16)};
          }
        }
      } else {
        // gate/up: h = silu(g) * u, rounded once
        if (!live) continue;
        const int to = WF ? ltok[MG * 32 + 32 * g] : 0;
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
          const int n = pair * 32 + vq * 8 + rq;
          uint16_t o[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float gv = a[0][vq][v], uv = a[NM - 1][vq][v];
            if constexpr (WF) {
              gv = __builtin_amdgcn_ldexpf(gv, lrow[8 * vq + v] - ts);
              uv = __builtin_amdgcn_ldexpf(uv, lrow[NWV * 32 + 8 * vq + v] - ts);
            }
            const float hv = silu_mul(gv, uv);
            o[v] = WF ? f32_to_f16_bits(__builtin_amdgcn_ldexpf(hv, to)) : f32_to_bf16(hv);
          }
          *(u32x2*)((uint16_t*)p.out + (size_t)m * p.N + n) =
              u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        }
      }
    }
  };
  auto own = [&](int mat, int g, int v4) {
    return f32x4{acc[mat][g][4 * v4], acc[mat][g][4 * v4 + 1], acc[mat][g][4 * v4 + 2], acc[mat][g][4 * v4 + 3]};
  };
  if (ks == 1) {
    rload();
    epilogue(own);
    return;
  }

  // Split tile, finished by last arrival: every piece publishes its whole partial tile in its
  // slot (tt, q) with write-through stores, waits for them and counts itself; the piece whose
  // count completes the tile (whichever it is) leaves the counter at zero, reads the ks partial
  // tiles -- its own among them -- and adds them in K order, p_0 + p_1 + ... + p_{ks-1}, so the
  // sum does not depend on the arrival order (deterministic), then runs the epilogue on every
  // group.  No piece waits for another.
  __shared__ int s_last;
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(p.part, 0, p.part_bytes, kBufferRsrcWord3);
  auto off = [&](int qq, int mat, int g, int v4) {  // byte offset of this lane's chunk in piece qq's slot
    return (uint32_t)(tt * ks + qq) * PART_BYTES + (uint32_t)((((wave * NM + mat) * MG + g) * 4 + v4) * 64 + lane) * 16u;
  };
#pragma unroll
  for (int mat = 0; mat < NM; ++mat)
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) store_coherent(prs, off(q, mat, g, v4), own(mat, g, v4));
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(p.counters + tt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == ks - 1;
    if (s_last) __hip_atomic_store(p.counters + tt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  rload();
  // every chunk's ks loads issued unconditionally, then added in K order
  auto fold = [&](auto ksc) {
    constexpr int KS = decltype(ksc)::value;
    epilogue([&](int mat, int g, int v4) {
      f32x4 v[KS];
#pragma unroll
      for (int r = 0; r < KS; ++r) v[r] = load_coherent(prs, off(r, mat, g, v4));
      f32x4 sum = v[0];
#pragma unroll
      for (int r = 1; r < KS; ++r) sum += v[r];
      return sum;
    });
  };
  static_assert(kSplitMaxPieces == 8, "fold instances");
  if (ks == 2)
    fold(std::integral_constant<int, 2>{});
  else if (ks == 3)
    fold(std::integral_constant<int, 3>{});
  else if (ks == 4 || NM == 2)  // the gate/up pair splits 4 ways at most
    fold(std::integral_constant<int, 4>{});
  else if constexpr (NM == 1) {
    if (ks == 5)
      fold(std::integral_constant<int, 5>{});
    else if (ks == 6)
      fold(std::integral_constant<int, 6>{});
    else if (ks == 7)
      fold(std::integral_constant<int, 7>{});
    else
      fold(std::integral_constant<int, 8>{});
  }
}

// ---------------------------------------------------------------- host side

constexpr int kTlNWV = 8;  // waves per block

// Block shapes (measured at the Qwen3-27B shape, 2048 tokens, bfp8):
//   gate/up: 1 tile per matrix per wave x 8 groups of 16 tokens (128 features x 128 tokens per
//            block): every dequantised weight fragment feeds 16 products (686-696 us, against
//            782-791 us for 2 tiles x 4 groups);
//   down:    2 tiles per wave x 4 groups (256 features x 64 tokens): 415-423 us, against 535-542
//            us for 1 tile x 8 groups, 488-492 us for 4 tiles x 4 groups, 424-437 us for 5.
// B register buffers (NBB): 3 where the registers allow two blocks per CU anyway or one block
// regardless (gate/up bfp8 704-707 us against 711-723; bf16 down 445 against 514 us; the bfp8
// down projection at 118 VGPRs once its loads went through buffer descriptors, 377 against 378).
constexpr int kTlGuTPW = 1, kTlGuMG = 8;
constexpr int kTlDnTPW = 2, kTlDnMG = 4;

// Resident blocks per CU of a kernel (its registers and LDS), once per kernel; 1 if unknown.
static int blocks_per_cu(const void* kern, size_t lds) {
  static std::mutex mu;
  static std::map<const void*, int> cache;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(kern);
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kTlNWV * 64, lds) != hipSuccess || n < 1) n = 1;
  cache[kern] = n;
  return n;
}

// Feature blocks [0, nbn) of a projection over token blocks of MG groups, as whole rounds of
// resident blocks where it pays: with nbn * nbm blocks and R resident at once, a last partial
// round leaves most CUs idle while it runs.  Then the first nbn_main feature blocks (a multiple of
// whole rounds) keep the block shape, and the remaining ones run on token blocks a quarter as
// tall (MGT groups), which fill a round of their own about four times faster.
static int tail_split(int nbn, int nbm, int rounds_of) {
  if (rounds_of < 1 || nbn * nbm <= rounds_of || (nbn * nbm) % rounds_of == 0) return nbn;
  int main = nbn;
  while (main > 0 && (main * nbm) % rounds_of) --main;
  return main;
}

template <int WF, int NMAT, int TPW, int MG, int NBB>
static int launch_tiled_part(TlParams p, int bn0, int nbn, int marks, hipStream_t s) {
  p.nbm = (p.M + MG * 16 - 1) / (MG * 16);
  p.bn0 = bn0;
  p.ks = 1;
  p.nfull = 0;
  const size_t lds = (size_t)3 * MG * 2048;
  launch_timed_part(NMAT == 2 ? 0 : 1, marks, tiled_kernel<WF, NMAT, TPW, MG, kTlNWV, NBB>, dim3(nbn * p.nbm),
                    dim3(kTlNWV * 64), lds, s, p);
  return check_launch("tiled_kernel");
}

// MGT: token groups of the tail launch (MGT == MG: no quarter-height tail).  The down projection
// (NMAT = 1) takes a K-split tail instead: its tail feature blocks keep their token blocks and
// split K into ks parts, whose partial tiles meet in the workspace (`part`, part_bytes), and
// these blocks follow the whole-K blocks in the same launch (`nfull`), so that each starts on
// the first CU slot to free up instead of after the last whole-K block.  A quarter-height tail
// re-reads every weight tile once per 16 tokens, which made the 27B down projection at 2048
// tokens slower (482 against 418 us).
template <int WF, int NMAT, int TPW, int MG, int NBB, int MGT>
static int launch_tiled(TlParams p, int num_cus, hipStream_t s) {
  const int nbn = p.N / (kTlNWV * TPW * kTileRows);
  const int nbm = (p.M + MG * 16 - 1) / (MG * 16);
  p.ks = 1;
  if constexpr (MGT == MG) {
    const int per_cu = blocks_per_cu((const void*)tiled_kernel<WF, NMAT, TPW, MG, kTlNWV, NBB>, (size_t)3 * MG * 2048);
    const int rounds_of = num_cus * per_cu;
    // fewer tiles than resident blocks (a few dozen to a few hundred tokens): every tile splits,
    // up to 8 ways (the last arrival adds the pieces one after another), into one block per CU
    // where that gives at least two pieces per tile, else into the resident slots (measured at the
    // 27B shape with bf16 weights: the down projection 61-85 us against 180-194 us at 33-256
    // tokens, 134 / 176 against 186 / 191 us at 512 / 768; filling the slots below 512 tokens
    // doubled blocks up on CUs: 87-102 us)
    const bool few = NMAT == 1 && p.part && nbn * nbm < rounds_of;
    const int main = few ? 0 : (NMAT == 1 && p.part ? tail_split(nbn, nbm, rounds_of) : nbn);
    const int tail_tiles = (nbn - main) * nbm;
    const size_t tile_bytes = (size_t)kTlNWV * TPW * MG * 256 * 4;
    int ks = tail_tiles > 0 ? std::min(std::max(1, rounds_of / tail_tiles), p.C) : 1;
    if (few && num_cus / tail_tiles >= 2) ks = std::min(num_cus / tail_tiles, p.C);
    if (few) ks = std::min(ks, 8);
    while (ks > 1 && (size_t)tail_tiles * ks * tile_bytes > (size_t)p.part_bytes) --ks;
    if (main == nbn || (main == 0 && !few) || ks < 2)
      return launch_tiled_part<WF, NMAT, TPW, MG, NBB>(p, 0, nbn, 3, s);
    p.ks = ks;
    p.nbm = nbm;
    p.bn0 = main;
    p.nfull = main * nbm;
    launch_timed_part(NMAT == 2 ? 0 : 1, 3, tiled_kernel<WF, NMAT, TPW, MG, kTlNWV, NBB>,
                      dim3(main * nbm + tail_tiles * ks), dim3(kTlNWV * 64), (size_t)3 * MG * 2048, s, p);
    return check_launch("tiled_kernel");
  }
  const int per_cu = blocks_per_cu((const void*)tiled_kernel<WF, NMAT, TPW, MG, kTlNWV, NBB>, (size_t)3 * MG * 2048);
  const int main = tail_split(nbn, nbm, num_cus * per_cu);
  if (main == nbn || main == 0) return launch_tiled_part<WF, NMAT, TPW, MG, NBB>(p, 0, nbn, 3, s);
  if (int rc = launch_tiled_part<WF, NMAT, TPW, MG, NBB>(p, 0, main, 1, s)) return rc;
  return launch_tiled_part<WF, NMAT, TPW, MGT, NBB>(p, main, nbn - main, 2, s);
}

// 32 x 32 gate/up kernel (block-float weights): 8 waves x 32 features x 4 groups of 32 tokens per
// block.  At 2048 tokens: bf4 (three B buffers) 676-692 against 711-739 us for tiled_kernel; bfp8
// (two B buffers, the next weight loads fenced behind the products) 721-723 against 732-737 us.
// bf16 weights stay on tiled_kernel (846-857 us here: the A stages spill).
constexpr int kTl32MG = 4;

// Bytes of one K piece's partial tile of tiled32_kernel (8 waves x NM 32-row units x MG groups of
// 32 tokens, fp32).
constexpr size_t split_part_bytes(int NM, int MG) { return (size_t)kTlNWV * NM * MG * 16 * 64 * 4; }

// Whole rounds plus K-split pieces for a tiled32 projection of ntiles tiles of C superblocks on
// `slots` resident blocks: the first rounds x slots tiles run whole; the remaining ntail tiles
// split K into ks <= 4 pieces with ntail x ks <= slots, so that the pieces fill at most one more
// round.  With fewer tiles than slots (a few dozen to a few hundred tokens) every tile splits, up
// to max_ks ways, its tiles rounded up to a multiple of 8 (whole XCDs; the padding blocks exit at
// once) so that each tile's pieces share an XCD.  ks = 1 (no split) where there is no remainder,
// where fewer than two pieces per tile fit, or where the workspace region does not hold the
// pieces' partial tiles.
struct SplitPlan {
  int nfull, ntail, ks;
  int npad;  // split tiles including the padding: the launch has nfull + npad x ks blocks
};
static SplitPlan split_plan(int ntiles, int C, int slots, size_t part_bytes, size_t piece_bytes, int max_ks) {
  const SplitPlan none{ntiles, 0, 1, 0};
  if (slots < 1) return none;
  const int rounds = ntiles / slots, ntail = ntiles - rounds * slots;
  if (ntail == 0 || 2 * (long long)ntail > kMaxDim / kTileRows) return none;
  const int npad = rounds ? ntail : (ntail + 7) / 8 * 8;
  int ks = std::min(std::min(slots / npad, C), rounds ? 4 : max_ks);
  while (ks > 1 && (size_t)ntail * ks * piece_bytes > part_bytes) --ks;
  if (ks < 2) return none;
  return {rounds * slots, ntail, ks, npad};
}

// Sized for the most any split can hold on kSplitMaxSlots resident blocks (one per CU of a 256-CU
// device) at every M that takes the many-token kernels: constant in M, so that the workspace never
// shrinks as M grows (the plan's own need does: 64 tail tiles at 2048 tokens, none at 2049).
// split_plan checks the size against the device's own block count at launch.
size_t tiled_split_bytes(int M, int H, int I, int fmt) {
  (void)H;
  (void)I;
  (void)fmt;  // bf16 weights: the down projection's split pieces (tiled_kernel) use the region too
  if (M <= 32) return 0;  // no many-token kernels
  return (size_t)kSplitMaxSlots * std::max(split_part_bytes(2, kTl32MG), split_part_bytes(1, kTl32MG));
}

// LDS of tiled32_kernel: the 3-slot B ring and the exponent staging area.
constexpr size_t tiled32_lds(int MG, int NM) { return (size_t)3 * MG * 4096 + (size_t)(NM * 256 + 2 * MG * 32) * 4; }

template <int WF, int MG, int NBB, int NM>
static int launch_tiled32_plan(TlParams p, int bn0, int nbm, const SplitPlan& sp, int slot, int marks,
                               hipStream_t s) {
  p.nbm = nbm;
  p.bn0 = bn0;
  p.nfull = sp.nfull;
  p.ntail = sp.ntail;
  p.ks = sp.ks;
  const size_t lds = tiled32_lds(MG, NM);
  launch_timed_part(slot, marks, tiled32_kernel<WF, MG, NBB, NM>, dim3(sp.nfull + sp.npad * sp.ks),
                    dim3(kTlNWV * 64), lds, s, p);
  return check_launch("tiled32_kernel");
}

// Gate/up: whole rounds plus K-split pieces in one launch where split_plan allows, else whole
// rounds of one tile per block plus a quarter-height tail launch.
template <int WF, int MG, int NBB>
static int launch_tiled32(TlParams p, int num_cus, hipStream_t s) {
  const int nbn = p.N / (kTlNWV * 2 * kTileRows);
  const int nbm = (p.M + MG * 32 - 1) / (MG * 32);
  const int slots = num_cus * blocks_per_cu((const void*)tiled32_kernel<WF, MG, NBB, 2>, tiled32_lds(MG, 2));
  const SplitPlan sp =
      p.part ? split_plan(nbn * nbm, p.C, slots, (size_t)p.part_bytes, split_part_bytes(2, MG), 4)
             : SplitPlan{0, 0, 1, 0};
  if (sp.ks > 1) return launch_tiled32_plan<WF, MG, NBB, 2>(p, 0, nbm, sp, 0, 3, s);
  const int main = tail_split(nbn, nbm, slots);
  if (main == nbn || main == 0)
    return launch_tiled32_plan<WF, MG, NBB, 2>(p, 0, nbm, {nbn * nbm, 0, 1, 0}, 0, 3, s);
  if (int rc = launch_tiled32_plan<WF, MG, NBB, 2>(p, 0, nbm, {main * nbm, 0, 1, 0}, 0, 1, s)) return rc;
  const int nbm1 = (p.M + 31) / 32;
  return launch_tiled32_plan<WF, 1, NBB, 2>(p, main, nbm1, {(nbn - main) * nbm1, 0, 1, 0}, 0, 2, s);
}

// bfp8 down projection on tiled32_kernel (NM = 1): each wave owns one 32-row unit x 4 groups of 32
// tokens, a block 256 features x 128 tokens, as whole rounds plus K-split pieces.  Returns 1
// (nothing launched) where that plan has no whole round or no split: then tiled_kernel runs the
// projection.
template <int MG>
static int launch_down32(TlParams p, int num_cus, hipStream_t s) {
  constexpr int NBB = 3;
  if (p.N % (kTlNWV * 2 * kTileRows)) return 1;
  const int nbn = p.N / (kTlNWV * 2 * kTileRows), nbm = (p.M + MG * 32 - 1) / (MG * 32);
  const int slots = num_cus * blocks_per_cu((const void*)tiled32_kernel<1, MG, NBB, 1>, tiled32_lds(MG, 1));
  const int ntiles = nbn * nbm;
  SplitPlan sp = p.part ? split_plan(ntiles, p.C, slots, (size_t)p.part_bytes, split_part_bytes(1, MG), 8)
                        : SplitPlan{ntiles, 0, 1, 0};
  if (sp.ks == 1 && !(ntiles >= slots && ntiles % slots == 0)) return 1;
  return launch_tiled32_plan<1, MG, NBB, 1>(p, 0, nbm, sp, 1, 3, s);
}

bool tiled_supported(int M, int H, int I) {
  return M >= 1 && I % (kTlNWV * kTlGuTPW * kTileRows) == 0 && H % (kTlNWV * kTlDnTPW * kTileRows) == 0;
}

int launch_forward_tiled(const ForwardArgs& a, int num_cus, hipStream_t s) {
  if (!tiled_supported(a.M, a.H, a.I)) return set_error(-1, "tiled path: H=%d I=%d not multiples of 256", a.H, a.I);
  const WsLayout L = ws_layout(a.M, a.H, a.I, a.fmt);
  const int fmt = a.fmt;
  int* tx = (int*)(a.ws + L.tx);
  int* th = (int*)(a.ws + L.th);
  uint16_t* x16 = (uint16_t*)(a.ws + L.x16);
  uint16_t* h = (uint16_t*)(a.ws + L.h);
  if (fmt != 0) {
    int rc = launch_prep(a, s);
    if (rc) return rc;
  }
  TlParams g{};
  g.w0 = a.wg;
  g.w1 = a.wu;
  g.rowexp0 = (const int*)(a.wg + rowexp_offset(a.I, a.H, fmt));
  g.rowexp1 = (const int*)(a.wu + rowexp_offset(a.I, a.H, fmt));
  g.src = fmt != 0 ? x16 : (const uint16_t*)a.x;
  g.M = a.M;
  g.K = a.H;
  g.N = a.I;
  g.C = a.H / kSuperK;
  g.tsrc = tx;
  g.tout = th;
  g.out = h;
  // partial tiles of the 32x32 kernels' K-split pieces: the region at xn (read only before the
  // gate/up projection, by the activation prep)
  g.part = L.split_bytes ? (float*)(a.ws + L.split) : nullptr;
  g.part_bytes = (int)std::min<size_t>(L.split_bytes, (size_t)1 << 30);
  g.counters = (int*)(a.ws + L.counters_gu);
  constexpr int GT = kTlGuTPW, GM = kTlGuMG, DT = kTlDnTPW, DM = kTlDnMG;
  // block-float: tiles of 2 groups of 32 tokens where that pads fewer token columns than tiles
  // of 4 (at most 256 tokens: up to 64 and from 129 to 192), of 4 otherwise.  Measured at the 27B
  // shape: 2 groups 111-113 against 269-275 us (the 4-group tiles before every tile split) at
  // 33-64 tokens, 162-166 against 194-196 us at 160-192; 4 groups 133 against 145 us at 96-128
  // and level at 224-256.
  const bool narrow = a.M <= 256 && (a.M + 63) / 64 * 64 < (a.M + 127) / 128 * 128;
  int rc = fmt == 2   ? (narrow ? launch_tiled32<2, 2, 3>(g, num_cus, s) : launch_tiled32<2, kTl32MG, 3>(g, num_cus, s))
           : fmt == 1 ? (narrow ? launch_tiled32<1, 2, 2>(g, num_cus, s) : launch_tiled32<1, kTl32MG, 2>(g, num_cus, s))
                      : launch_tiled<0, 2, GT, GM, 2, GM / 4>(g, num_cus, s);
  if (rc) return rc;
  TlParams d{};
  d.w0 = a.wd;
  const int dfmt = down_format(fmt);
  d.rowexp0 = (const int*)(a.wd + rowexp_offset(a.H, a.I, dfmt));
  d.src = h;
  d.M = a.M;
  d.K = a.I;
  d.N = a.H;
  d.C = a.I / kSuperK;
  d.tsrc = th;
  d.out = a.out;
  d.residual = a.residual;
  d.out_f32 = a.out_f32;
  d.res_f32 = a.res_f32;
  // the K-split tail's partial tiles: x16 and xn (adjacent, read only by the gate/up projection)
  d.part = (float*)(a.ws + L.x16);
  d.part_bytes = (int)std::min<size_t>(L.total - L.x16, (size_t)1 << 30);
  d.counters = (int*)(a.ws + L.counters_d);
  if (dfmt == 1) {
    TlParams d32 = d;
    d32.part = L.split_bytes ? (float*)(a.ws + L.split) : nullptr;
    d32.part_bytes = (int)std::min<size_t>(L.split_bytes, (size_t)1 << 30);
    d32.counters = (int*)(a.ws + L.counters_d);
    rc = narrow ? launch_down32<2>(d32, num_cus, s) : launch_down32<kTl32MG>(d32, num_cus, s);
    if (rc != 1) return rc;
  }
  rc = dfmt == 1 ? launch_tiled<1, 1, DT, DM, 3, DM>(d, num_cus, s) : launch_tiled<0, 1, DT, DM, 3, DM>(d, num_cus, s);
  if (rc) return rc;
  return 0;
}

}  // namespace qmlp
