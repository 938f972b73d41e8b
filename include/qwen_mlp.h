/*
 * qwen_mlp.h -- C ABI of libqwen_mlp.so, the MI355X (gfx950) fused Qwen3 SwiGLU MLP.
 *
 *   out = residual + down( silu(gate(x)) * up(x) )          (residual optional)
 *
 * Every pointer is a device pointer unless stated otherwise; every buffer is owned by the caller;
 * the library never allocates or frees device memory.  Work is enqueued on the given HIP stream
 * (nullptr = the legacy default stream), nothing synchronises the host unless stated, and no
 * call allocates, so the forward entry points can be captured in a HIP graph.
 *
 * Return codes: QMLP_OK (0) or a negative QMLP_E_* code; qmlp_last_error() then returns a
 * thread-local message naming the failing argument.
 *
 * Weight formats:
 *   QMLP_FMT_BF16  bf16 weights, bf16 matrix-core products, fp32 accumulation.
 *   QMLP_FMT_BFP8  bfp8 block float: 16 consecutive K values share one 8-bit exponent, each value
 *                  1 sign + 7 magnitude bits; dequantised in registers to fp16 matrix-core
 *                  operands, fp32 accumulation.
 *   QMLP_FMT_BF4   bf4 block float: the same 16-value groups with 1 sign + 3 magnitude bits
 *                  (0.5625 B/value).  In qmlp_forward it names the reference's mixed layout
 *                  (mlp.py:17-19,164-169): gate_proj and up_proj packed bf4, down_proj packed bfp8.
 * Weights are used in the library's packed ("tiled") layout, produced once by qmlp_pack().
 * Matrices are row-major [out_features, in_features] like the HF checkpoint tensors
 * gate_proj.weight [I,H], up_proj.weight [I,H], down_proj.weight [H,I].
 */
#ifndef QWEN_MLP_H
#define QWEN_MLP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* qmlp_stream_t; /* == hipStream_t */

#define QMLP_OK 0
#define QMLP_E_SHAPE (-1)     /* bad dimension (H, I, M, rows, cols) */
#define QMLP_E_ALIGN (-2)     /* pointer not 16-byte aligned */
#define QMLP_E_FORMAT (-3)    /* unknown format, or packed data that does not fit the format */
#define QMLP_E_LAUNCH (-4)    /* HIP launch / runtime error */
#define QMLP_E_WORKSPACE (-5) /* workspace too small */
#define QMLP_E_NULL (-6)      /* required pointer is null */
#define QMLP_E_DEVICE (-7)    /* no usable gfx950 device */

#define QMLP_FMT_BF16 0
#define QMLP_FMT_BFP8 1
#define QMLP_FMT_BF4 2

/* Message for the last failing call on this host thread ("" if none).  Host only. */
const char* qmlp_last_error(void);

/* Library version string, "qwen_mlp <version> gfx950 src=<digest>": the digest (16 hex digits) is
 * the sha256 of the kernel sources and this header that the build compiled.  Host only. */
const char* qmlp_version(void);

/* ---------------------------------------------------------------- weight preparation (load time)
 *
 * The reference converts host bf16 tensors into device block-float tiles once per model
 * (docker/qwen-c2-graft/graft/mlp.py:125-169, ttnn.as_tensor(..., dtype=bfloat8_b/bfloat4_b,
 * layout=TILE_LAYOUT)); these calls are that step.
 */

/* Canonical bfp8 quantisation of a bf16 matrix w[rows, cols] (row-major, K = cols).
 * q: int8 [rows, cols]; e8: uint8 [rows, cols/16] (scale 2^(e8-127), 0 = zero group).
 * bad_groups (device uint32, nullable): incremented once per group holding a non-finite value.
 * Replaces the host quantiser inside ttnn.as_tensor(dtype=bfloat8_b) (mlp.py:155-162). */
int qmlp_quantize_bfp8(const void* w_bf16, int rows, int cols, void* q, void* e8,
                       uint32_t* bad_groups, qmlp_stream_t stream);

/* Canonical bf4 quantisation: as qmlp_quantize_bfp8 with magnitudes in [0, 7] (q in [-7, 7],
 * scale 2^(e8-127) with e8 = exponent of the group maximum + 127 - 3).  Replaces the host
 * quantiser inside ttnn.as_tensor(dtype=bfloat4_b) (mlp.py:17-19,164-169). */
int qmlp_quantize_bf4(const void* w_bf16, int rows, int cols, void* q, void* e8,
                      uint32_t* bad_groups, qmlp_stream_t stream);

/* Bytes of the packed device buffer for one [rows, cols] matrix (host only, no GPU needed). */
size_t qmlp_packed_bytes(int rows, int cols, int fmt);

/* Pack one matrix into the library's tiled layout.
 *   fmt == QMLP_FMT_BFP8 or QMLP_FMT_BF4: src0 = q (int8 [rows,cols]), src1 = e8 (uint8
 *   [rows,cols/16]) from the matching quantiser.
 *   fmt == QMLP_FMT_BF16: src0 = bf16 [rows,cols], src1 unused (may be null).
 * packed must hold qmlp_packed_bytes(rows, cols, fmt) bytes.  The trailer of the packed buffer
 * records the largest row L2 norm and the number of bfp8 groups too small to keep (see
 * qmlp_packed_info); a nonzero count means the packed matrix is not lossless.
 * Replaces _build_gate_up / load_mlp_weights' tile conversion (mlp.py:23-42, 125-169). */
int qmlp_pack(const void* src0, const void* src1, int rows, int cols, int fmt, void* packed,
              size_t packed_bytes, qmlp_stream_t stream);

/* Reads the packed trailer back to host memory: largest row L2 norm (of the dequantised rows)
 * and count of flushed bfp8 groups.  Synchronises `stream`.  Load-time only. */
int qmlp_packed_info(const void* packed, int rows, int cols, int fmt, double* max_row_norm,
                     uint32_t* flushed_groups, qmlp_stream_t stream);

/* Inverse of qmlp_pack for bfp8 (lossless for every group that was not flushed): packed ->
 * canonical q/e8.  Used by the on-disk weight cache and the packing audit (the reference audits
 * its packed gate/up the same way, packed_weight_check.cpp:1-37). */
int qmlp_unpack_bfp8(const void* packed, int rows, int cols, void* q, void* e8,
                     qmlp_stream_t stream);

/* Inverse of qmlp_pack for bf4 (same contract as qmlp_unpack_bfp8). */
int qmlp_unpack_bf4(const void* packed, int rows, int cols, void* q, void* e8,
                    qmlp_stream_t stream);

/* Dequantises a packed matrix to fp32 [rows, cols] with the same in-register routine the GEMM
 * kernels use.  Diagnostic/audit use. */
int qmlp_dequant_packed(const void* packed, int rows, int cols, int fmt, float* out,
                        qmlp_stream_t stream);

/* ---------------------------------------------------------------- forward (hot path)
 *
 * Replaces Qwen36MLP.forward(x) (docker/qwen-c2-graft/graft/mlp.py:402-423) and, at M = 16, the
 * reference's fused route FusedT16Arm.forward (scripts/ci/fused_t16_scope.py:45-76):
 * FusedProjection (scripts/ci/fused_1d.py:123-196) + down linear (fused_t16_scope.py:64-67);
 * the residual add of Qwen36DecoderLayer.forward (layer.py:357) is fused when residual != null.
 *
 *   x        bf16 [M, H] row-major
 *   wg, wu   packed [I, H] (gate_proj, up_proj); wd packed [H, I] (down_proj); all in fmt, except
 *            that fmt == QMLP_FMT_BF4 takes wd packed QMLP_FMT_BFP8
 *   residual bf16 [M, H] or null
 *   out      bf16 [M, H]; may alias residual (each element is read before it is written by the
 *            same thread) but must not alias x
 *   ws       workspace of at least qmlp_workspace_bytes(M, H, I, fmt) bytes, initialised once by
 *            qmlp_workspace_init; the kernels leave it re-usable.  Concurrent forwards need
 *            separate workspaces.
 * Constraints: H and I multiples of 256; 1 <= M <= 65536 and M * max(H, I) < 2^30; pointers
 * 16-byte aligned.
 * M <= 32 uses the weight-streaming kernels; larger M the LDS-tiled matrix-core kernels. */
int qmlp_forward(const void* x, const void* wg, const void* wu, const void* wd,
                 const void* residual, void* out, void* ws, size_t ws_bytes, int M, int H, int I,
                 int fmt, qmlp_stream_t stream);

/* qmlp_forward with options.  flags: QMLP_OUT_F32 -- out is fp32 [M, H] (the fp32 sum
 * residual + y, not rounded); QMLP_RESIDUAL_F32 -- residual is fp32 [M, H] (an fp32 residual
 * stream).  qmlp_forward(...) == qmlp_forward_ex(..., 0, stream). */
#define QMLP_OUT_F32 1
#define QMLP_RESIDUAL_F32 2
int qmlp_forward_ex(const void* x, const void* wg, const void* wu, const void* wd,
                    const void* residual, void* out, void* ws, size_t ws_bytes, int M, int H, int I,
                    int fmt, int flags, qmlp_stream_t stream);

/* The decoder's feed-forward half with its RMSNorm prologue:
 *
 *   out = h + down( silu(gate(n)) * up(n) ),   n = h / sqrt(mean(h^2) + eps) * (1 + norm_w)
 *
 * (the zero-centred RMSNorm, mean over H).  Replaces ff_input = self.ffn_norm(h);
 * ff_output = self.feed_forward.forward(ff_input); output = ttnn.add(h, ff_output)
 * (docker/qwen-c2-graft/graft/layer.py:352-357; the norm is the framework RMSNorm with
 * add_unit_offset, layer.py:110-112,228-237).
 *   h       bf16 [M, H], the pre-norm hidden state (also the residual)
 *   norm_w  bf16 [H]
 *   out     bf16 [M, H] (fp32 with QMLP_OUT_F32); may equal h (in-place residual update)
 * Other arguments and constraints as qmlp_forward_ex (QMLP_RESIDUAL_F32 is not accepted).  n is
 * rounded to bf16, as the reference's separate norm writes it.  M <= 32 fuses the norm into the
 * gate/up kernel's activation staging (each workgroup reduces the whole row's sum of squares in
 * one fixed order, so every K range of a token sees the same 1/rms); larger M (and the long-K
 * fallback) run it as one extra pass over h. */
int qmlp_forward_rmsnorm(const void* h, const void* norm_w, float eps, const void* wg, const void* wu,
                         const void* wd, void* out, void* ws, size_t ws_bytes, int M, int H, int I,
                         int fmt, int flags, qmlp_stream_t stream);

/* Workspace bytes needed by qmlp_forward for these sizes (host only, no GPU needed).  The size
 * never decreases as M grows, so a workspace sized for M serves every call with fewer tokens, and
 * one workspace serves calls of different shapes as long as it is large enough for each. */
size_t qmlp_workspace_bytes(int M, int H, int I, int fmt);

/* The first QMLP_WS_COUNTER_BYTES bytes of every workspace hold arrival counters, at the same
 * place for every shape.  They must read zero when a forward starts, and every forward leaves them
 * zero.  The rest of the workspace may hold anything when a forward starts. */
#define QMLP_WS_COUNTER_BYTES 524288

/* Zero-fills the workspace with a kernel (not a memset node, so it may be graph-captured). */
int qmlp_workspace_init(void* ws, size_t ws_bytes, qmlp_stream_t stream);

/* qmlp_forward_ex without a workspace argument.  No counterpart in the reference: this entry point
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The workspace is a QMLP_SCRATCH_BYTES array of device
 * memory inside the library, one per GPU, held until the process ends; the call allocates and
 * frees nothing.  It serves every call whose qmlp_workspace_bytes(M, H, I, fmt) fits, e.g. M <= 32
 * at H = 5120, I = 17408; larger calls fail with QMLP_E_WORKSPACE.  The array starts zeroed (it
 * is loaded with the library's code object), and every forward leaves its arrival counters at
 * zero.  The first call on a device looks up the array's address (hipGetSymbolAddress) and must
 * be made outside graph capture: a first call on a capturing stream fails with QMLP_E_LAUNCH;
 * later calls may be captured.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (several streams or host threads) race and must be serialised by the caller.
 * Arguments, constraints and results as qmlp_forward_ex. */
#define QMLP_SCRATCH_BYTES 33554432
int qmlp_forward_noalloc(const void* x, const void* wg, const void* wu, const void* wd,
                         const void* residual, void* out, int M, int H, int I, int fmt, int flags,
                         qmlp_stream_t stream);

/* ---------------------------------------------------------------- profiling (host only)
 *
 * Per-kernel timing of the forward pass, the counterpart of the reference's per-op signposts
 * (docker/qwen-c2-graft/graft/layer.py:18-90).  When n == 4, every later qmlp_forward on this host
 * thread launches its gate/up kernel with events[0] / events[1] as the start / stop events of
 * hipExtLaunchKernel and its down kernel with events[2] / events[3] (hipEvent_t handles): each
 * pair then holds the timestamps of that dispatch itself, and no marker packets are inserted
 * between the kernels.  n == 0 turns timing off.  Kernels outside the two projections (the
 * RMSNorm pass, the prefill's activation prep) are not timed. */
int qmlp_set_profile_events(void* const* events, int n);

/* ---------------------------------------------------------------- planning (host only)
 *
 * Work split of the M <= 32 stream-K kernel (the fallback where qmlp_plan_split finds no split)
 * for one projection: `rows` output rows (multiple of 16) over K (multiple of 256) on `num_cus`
 * compute units.  Fills out[0..1] =
 * {workgroups, tiles one wave may touch}.  Exposed so the coverage of the split can be tested
 * without a GPU, like the reference's worker-to-pair mapping tests
 * (scripts/ci/test_fused_1d.py:71-79). */
int qmlp_plan_stream(int rows, int K, int num_cus, int* out2);

/* Work split of the M <= 32 weight-streaming kernel for one projection with `nmat` matrices
 * (2 = gate/up, 1 = down) at M tokens (1..32; 17..32 run as two groups of 16): the (16-row tile
 * x 256-K superblock) grid cut into tile groups x K splits, split q covering superblocks
 * [q*C/S, (q+1)*C/S) of C = K/256.  Fills out[0..5] = {workgroups, tiles per group, K splits,
 * superblocks of the longest split, groups, tiles one wave may touch}. */
int qmlp_plan_split(int rows, int K, int nmat, int M, int num_cus, int* out6);

#ifdef __cplusplus
}
#endif

#endif /* QWEN_MLP_H */
