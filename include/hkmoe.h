/*
 * hkmoe.h -- C ABI of the MI355X (gfx950) FP8 mixture-of-experts path.
 *
 * Plain pointers and sizes only (no torch types).  Every entry point:
 *   - takes device pointers that the caller owns (outputs preallocated, as the
 *     reference's dispatch functions expect: C is allocated by the caller in
 *     kernels/cdna3/gemm/fp8fp32/mi300x/8192_256_256_64_32/data_logs/
 *     0613_003858_outputs/test_python.py:12);
 *   - enqueues asynchronously on `stream` (a hipStream_t; NULL = the null
 *     stream) and never synchronises with the host; per-expert offsets stay on
 *     the device;
 *   - returns HKMOE_OK or an error code; hkmoe_last_error() then describes the
 *     failure (thread-local).  Shape/size errors are detected on the host
 *     before anything is launched, mirroring the std::runtime_error checks of
 *     include/pyutils/pyutils.cuh:17-45.
 *
 * Formats: e4m3 = OCP float8 e4m3fn bytes; bf16 = bfloat16 bits; scales fp32.
 * Tensor layouts are row-major; "[K/128, ld]" marks the transposed activation
 * scale layout used inside the layer's workspace.
 */
#ifndef HKMOE_H
#define HKMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* hkmoe_stream_t; /* hipStream_t */

enum hkmoe_status {
  HKMOE_OK = 0,
  HKMOE_ERR_INVALID_ARGUMENT = 1,
  HKMOE_ERR_UNSUPPORTED = 2,
  HKMOE_ERR_HIP = 3,
  HKMOE_ERR_WORKSPACE = 4
};

enum hkmoe_dtype { HKMOE_BF16 = 0, HKMOE_F32 = 1, HKMOE_E4M3 = 2 };

enum hkmoe_scale_mode {
  HKMOE_SCALE_TENSOR = 0, /* one fp32 scale per tensor (weights: one per expert) */
  HKMOE_SCALE_BLOCK = 1,  /* activations 1x128 groups, weights 128x128 blocks */
  HKMOE_SCALE_MX = 2      /* 1x32 e8m0 exponents on both operands (MX layer entry points) */
};

/* Byte layout of expert weights [E, N, K] given to the grouped GEMMs. */
enum hkmoe_weight_layout {
  HKMOE_W_ROWS = 0,  /* row-major [E, N, K] */
  HKMOE_W_PACKED = 1 /* hkmoe_pack_weights output (same size) */
};

/* Library version (major*10000 + minor*100 + patch) and last error text. */
int hkmoe_version(void);
const char* hkmoe_last_error(void);

/*
 * Dense FP8 GEMM  C[M,N] = (sa*sb) * sum_k A[m,k] * B[n,k]   (A . B^T, "TN")
 *   A [M,K] e4m3, B [N,K] e4m3, C [M,N] bf16 (RNE) or fp32.
 *   scale_a, scale_b: device fp32 scalars, or NULL for 1.0.
 *   Requires K % 128 == 0 and N % 256 == 0; M is arbitrary.
 * Replaces the reference's dispatch_micro(A, B, C) (C = A . B^T, fp32 out):
 *   kernels/cdna3/gemm/fp8fp32/mi300x/8192_256_256_64_32/data_logs/
 *   0613_003858_outputs/256_256_64_32.cpp:202-212 and the FP8 GEMM kernels named
 *   by kernels/cdna4/gemm/fp8fp32/FP8_4wave/Makefile:5 (sources absent there).
 */
int hkmoe_gemm_fp8(const void* a, const void* b, void* c, int64_t m, int64_t n, int64_t k,
                   const float* scale_a, const float* scale_b, int out_dtype,
                   hkmoe_stream_t stream);

/*
 * MFMA shape of hkmoe_gemm_fp8's kernel for small problems (fewer 256x256 tiles
 * than two per CU, e.g. 2048^3), which runs 128x128 tiles: 16 for
 * v_mfma_f32_16x16x128_f8f6f4, 32 for v_mfma_f32_32x32x64_f8f6f4 (the default:
 * 4-7% faster at 2048^3 and similar shapes).
 * Both give the same sums (fp32 accumulation in another order).  Replaces the
 * choice between the reference's mfma1616128 and mfma323264 wrappers
 * (include/cdna4/ops/warp/register/tile/mma.cuh:97-125).  Other values are
 * rejected; the setting is process-wide.
 */
int hkmoe_set_dense_mfma(int32_t shape);
int hkmoe_get_dense_mfma(void);

/*
 * Routing step 1: top-k + softmax weights + per-block expert histogram.
 *   logits [T,E] fp32 -> topk_idx [T,k] int32, topk_w [T,k] fp32.
 *   Order: descending logit, ties to the lower expert id.  Weights: softmax
 *   over the k selected logits.  block_counts: workspace [nblk, E] int32 with
 *   nblk = hkmoe_route_blocks(T).  E <= 1024, 1 <= k <= min(E, 32).
 * The reference has no router, histogram or permutation: the routing entry
 * points (this one, hkmoe_expert_offsets, hkmoe_scatter) and the MoE entry
 * points below have no reference counterpart; they follow its binding style
 * (caller-owned device buffers, one call per kernel as in dispatch_micro).
 */
int hkmoe_route_blocks(int64_t num_tokens);
int hkmoe_route_topk(const float* logits, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                     int32_t* topk_idx, float* topk_w, int32_t* block_counts,
                     hkmoe_stream_t stream);

/*
 * Routing step 2: expert offsets.  From block_counts [nblk, E] computes
 *   counts [E], offsets [E+1] (exclusive prefix sum, offsets[E] = T*k),
 *   block_base [nblk, E] (rows of expert e routed from earlier blocks),
 *   mtile_offsets [E+1] (prefix sum of ceil(counts/256): the grouped GEMM's
 *   M-tile list), and zeroes *amax_reset and the HKMOE_TILE_COUNTERS ints at
 *   tile_counters when they are non-NULL.
 *   mtile_list (may be NULL): [ceil(T*k/256) + E][2] int32; receives one
 *   (expert, first row) pair per M tile: first every expert with at least one
 *   full 256-row tile, with all its tiles (expert order), then the single
 *   partial tiles of the smaller experts.  Passed to the grouped
 *   GEMMs it sets their tile order (tiles of equal cost run together, which
 *   keeps L2 reuse up); NULL there means expert order.
 */
#define HKMOE_TILE_COUNTERS 16 /* 8 per grouped GEMM: one tile queue per XCD */
int hkmoe_expert_offsets(const int32_t* block_counts, int64_t num_tokens, int32_t num_experts,
                         int32_t* counts, int32_t* offsets, int32_t* block_base,
                         int32_t* mtile_offsets, int32_t* mtile_list, float* amax_reset,
                         int32_t* tile_counters, hkmoe_stream_t stream);

/*
 * Routing step 3: stable scatter into expert-contiguous order.
 *   perm [T*k]: perm[p] = t*k + j (f ascending within an expert);
 *   inv_perm [T*k]: inv_perm[t*k+j] = p.
 *   When x_q is non-NULL also gathers rows: xp[p] = x_q[perm[p] / k] ([T*k, H]
 *   e4m3) and, for HKMOE_SCALE_BLOCK, xp_scale_t[g, p] = x_scale[perm[p]/k, g]
 *   (transposed [H/128, T*k]).
 */
int hkmoe_scatter(const int32_t* topk_idx, int64_t num_tokens, int32_t num_experts, int32_t top_k,
                  const int32_t* offsets, const int32_t* block_base, int32_t* perm,
                  int32_t* inv_perm, const void* x_q, const float* x_scale, int64_t hidden,
                  int scale_mode, void* xp, float* xp_scale_t, hkmoe_stream_t stream);

/*
 * Grouped GEMM 1 with fused SiLU(gate)*up:
 *   h[p, i] = bf16( silu(g) * u ),  [g | u] = deq(x[row(p)]) . deq(W13[e])^T
 *   for every row p of expert e (rows ordered by expert, offsets [E+1]).
 *   x [x_rows, H] e4m3; row(p) = gather[p] / gather_div when gather != NULL
 *   (the expert-sorted permutation: token rows are read in place, no permuted
 *   copy), else row(p) = p.
 *   w13 [E, 2I, H] e4m3 (gate rows 0..I-1, up rows I..2I-1).
 *   TENSOR: x_scale [1], w13_scale [E]; out_format must be HKMOE_BF16:
 *           h bf16 [rows, I], and max|h| is accumulated into h_aux[0] (must be
 *           zeroed before; hkmoe_expert_offsets can do it; may be NULL).
 *   BLOCK:  x_scale [x_rows, H/128], w13_scale [E, 2I/128, H/128];
 *           out_format HKMOE_BF16: h bf16 [rows, I] (h_aux unused), or
 *           out_format HKMOE_E4M3: the 1x128-group requantisation of that bf16 h
 *           is fused in: h e4m3 [rows, I], h_aux = group scales [I/128, rows].
 *   w_layout: HKMOE_W_ROWS, or HKMOE_W_PACKED for w13 packed by
 *   hkmoe_pack_weights(..., gate_up = I) (same results, bit for bit).
 *   mtile_list: NULL (expert order) or the list written by hkmoe_expert_offsets.
 *   tile_counters: NULL (static tile order) or 8 zeroed ints, consumed by the
 *   call (per-XCD tile queues keep ragged tiles L2-local; zero before reuse).
 *   Requires H % 128 == 0, I % 128 == 0, H <= 16384.
 */
int hkmoe_grouped_gemm1(const void* x, const float* x_scale, const int32_t* gather,
                        int32_t gather_div, int64_t x_rows, const void* w13,
                        const float* w13_scale, const int32_t* offsets,
                        const int32_t* mtile_offsets, const int32_t* mtile_list,
                        int64_t rows, int32_t num_experts,
                        int32_t hidden, int32_t inter, int scale_mode, int w_layout,
                        int out_format, void* h, float* h_aux, int32_t* tile_counters,
                        hkmoe_stream_t stream);

/*
 * Requantise a bf16 intermediate to e4m3 for GEMM 2.
 *   TENSOR: hs[0] = scale(amax), hq = e4m3(h / hs[0]) (amax from GEMM 1).
 *   BLOCK:  1x128 groups, hs_t [I/128, R] (transposed) = scale(amax_g).
 *   scale(a) = max(a / 448, 2^-126), or 1 for a == 0 (and for a NaN a).
 *   A NaN h gives +-448 (0x7E | sign) rather than the NaN code.
 */
int hkmoe_requant(const void* h, int64_t rows, int32_t inter, int scale_mode, const float* amax,
                  void* hq, float* hs, hkmoe_stream_t stream);

/*
 * Grouped GEMM 2:  y[p] = bf16( deq(hq[p]) . deq(W2[e])^T ),  w2 [E, H, I].
 *   TENSOR: hs [1], w2_scale [E];  BLOCK: hs_t [I/128, R], w2_scale [E, H/128, I/128].
 *   w_layout: HKMOE_W_ROWS, or HKMOE_W_PACKED (hkmoe_pack_weights, gate_up = 0).
 *   mtile_list, tile_counters: as for hkmoe_grouped_gemm1.
 *   Requires H % 256 == 0, I % 128 == 0.
 */
int hkmoe_grouped_gemm2(const void* hq, const float* hs, const void* w2, const float* w2_scale,
                        const int32_t* offsets, const int32_t* mtile_offsets,
                        const int32_t* mtile_list, int64_t rows,
                        int32_t num_experts, int32_t hidden, int32_t inter, int scale_mode,
                        int w_layout, void* y, int32_t* tile_counters, hkmoe_stream_t stream);

/*
 * The same layer split for the narrow path of hkmoe_moe_forward (block scales,
 * e4m3 h), for callers that enqueue the parts themselves:
 *   hkmoe_expert_offsets_narrow: hkmoe_expert_offsets that also moves the experts
 *     of 1..narrow_max rows (narrow_max <= 64) to the end of the M-tile list,
 *     writes their count to narrow_info[0] and zeroes the narrow kernels'
 *     counters narrow_info[1..4] (narrow_info: 5 int32 of device memory).
 *   hkmoe_grouped_gemm{1,2}_part: part 0 runs the 256x256 kernel on the list
 *     without those experts, one workgroup per CU; when narrow experts exist,
 *     its workgroups from `grid` on exit at once and leave their CUs to part 1
 *     (grid 0: none do).  Part 1 runs the narrow kernel on exactly those
 *     experts, one workgroup per CU, of which the first `grid` to start take
 *     items (0: all of them) while the list also holds 256x256 tiles; its
 *     counters are narrow_info[1] and [3] for GEMM 1, [2] and [4] for GEMM 2,
 *     so it runs once per
 *     hkmoe_expert_offsets_narrow (tile_counters is not used), and its K steps
 *     per item, H/128 or I/128, must be even and at most 64.  The two parts write disjoint
 *     rows and may run concurrently on two streams;
 *     together they give the bits of hkmoe_grouped_gemm{1,2}.
 * No reference counterpart (the reference has no grouped GEMM).
 */
int hkmoe_expert_offsets_narrow(const int32_t* block_counts, int64_t num_tokens, int32_t num_experts,
                                int32_t* counts, int32_t* offsets, int32_t* block_base,
                                int32_t* mtile_offsets, int32_t* mtile_list, float* amax_reset,
                                int32_t* tile_counters, int32_t narrow_max, int32_t* narrow_info,
                                hkmoe_stream_t stream);
int hkmoe_grouped_gemm1_part(const void* x, const float* x_scale, const int32_t* gather,
                             int32_t gather_div, int64_t x_rows, const void* w13, const float* w13_scale,
                             const int32_t* offsets, const int32_t* mtile_offsets,
                             const int32_t* mtile_list, int64_t rows, int32_t num_experts, int32_t hidden,
                             int32_t inter, int w_layout, void* hq, float* hs, int32_t* tile_counters,
                             const int32_t* narrow_info, int32_t part, int32_t grid, hkmoe_stream_t stream);
int hkmoe_grouped_gemm2_part(const void* hq, const float* hs, const void* w2, const float* w2_scale,
                             const int32_t* offsets, const int32_t* mtile_offsets, const int32_t* mtile_list,
                             int64_t rows, int32_t num_experts, int32_t hidden, int32_t inter, int w_layout,
                             void* y, int32_t* tile_counters, const int32_t* narrow_info, int32_t part,
                             int32_t grid, hkmoe_stream_t stream);

/*
 * Load-time weight packing for the grouped GEMMs: w [E, N, K] e4m3 row-major
 * -> packed (E*N*K bytes, another buffer).  Every 256-row N tile x 128-byte
 * K step becomes one contiguous 32 KiB block holding its sixteen 16-row MFMA
 * fragments in operand-register order (each fragment as two 1 KiB register
 * halves: byte f*2048 + h*1024 + l*16 + b = row 16f + l%16, K byte
 * (2*(l/16) + h)*16 + b); block (e, kt, nt) sits at ((e*(K/128) + kt)*(N/256)
 * + nt)*32 KiB, so every 64-lane load of a register half reads 1 KiB of whole
 * cache lines and the N tiles of one K step are adjacent.  gate_up = I for the fused gate/up
 * weights of GEMM 1 (N = 2I: rows [gate | up]), 0 otherwise.
 * Requires N % 256 == 0, K % 128 == 0 (gate_up: N == 2*gate_up).
 * No reference counterpart (the reference's GEMMs read [N, K] rows directly);
 * it plays the role of a checkpoint-load weight shuffle.
 */
int hkmoe_pack_weights(const void* w, int64_t num_experts, int64_t n, int64_t k, int32_t gate_up,
                       void* packed, hkmoe_stream_t stream);

/*
 * Self-check of the requantisation quotient used by the GEMM 1 epilogues
 * (256x256 and narrow kernels): each value x of a 1x128 group is divided by its
 * scale s without a division per value (x and s scaled by one power of two so
 * that s is in [1, 2), fl(x*y) with y = fl(1/s), one exact-remainder FMA
 * correction).  This launches one kernel that compares the result with the
 * IEEE quotient x / s over every input those epilogues can produce (x a bf16
 * value, s = max(amax/448, 2^-126) with amax a bf16 value >= |x|; mantissas
 * exhaustive, exponents sampled, both signs, bf16 subnormals and signed zeros,
 * amax = inf):
 * the e4m3 bytes must agree, and the fp32 quotients wherever |x/s| >= 2^-10.
 * counts [2] int32 on the device, zeroed by the caller: counts[0] += cases,
 * counts[1] += mismatches.
 * No reference counterpart (the reference has no requantisation step).
 */
int hkmoe_requant_quotient_check(int32_t* counts, hkmoe_stream_t stream);

/*
 * Top-k weighted unpermute/combine:
 *   out[t] = bf16( sum_{j<k} topk_w[t,j] * y[inv_perm[t*k+j]] ), fp32 accumulate.
 *   y [T*k, H] bf16, out [T, H] bf16, H % 8 == 0.
 */
int hkmoe_combine(const void* y, const float* topk_w, const int32_t* inv_perm, int64_t num_tokens,
                  int32_t top_k, int32_t hidden, void* out, hkmoe_stream_t stream);

/*
 * Whole layer: route -> scatter -> GEMM1+SiLU*up -> requant -> GEMM2 -> combine.
 *   x_q [T,H] e4m3; x_scale [1] (TENSOR) or [T, H/128] (BLOCK);
 *   logits [T,E] fp32; w13/w2 and scales as above, both in w_layout; out [T,H]
 *   bf16.  workspace: device buffer of hkmoe_moe_workspace_size(...) bytes,
 *   256-byte aligned, holding every intermediate (routing, permutation, h, y).
 *   hkmoe_moe_workspace_size also sizes hkmoe_moe_forward_mx's workspace with
 *   scale_mode HKMOE_SCALE_MX (0 for an unknown mode).
 *   T == 0: weights and shapes are checked, nothing is launched, and x_q,
 *   x_scale (block), logits, out and the workspace may be null (the same for
 *   hkmoe_moe_forward_mx and hkmoe_moe_forward_noalloc).
 */
size_t hkmoe_moe_workspace_size(int64_t num_tokens, int32_t num_experts, int32_t top_k,
                                int32_t hidden, int32_t inter, int scale_mode);
/*
 * Narrow path of hkmoe_moe_forward (block scales only): the experts with
 * 1..max_rows rows (max_rows <= 64) go to a weight-streaming grouped GEMM
 * (both GEMMs) that runs on `cus` workgroups on a library-owned auxiliary
 * stream, beside the 256x256 kernels of the larger experts on the caller's
 * stream; the caller's stream waits for it before the combine.  Results are
 * bit-identical with the narrow path on or off.  cus == 0 turns it off; while
 * 256x256 tiles exist the narrow kernels take at most three quarters of the
 * device's CUs, whatever cus asks for (the first wide GEMM keeps the rest);
 * wide_share 1 or 2 runs the first wide GEMM on (CUs - cus) workgroups while
 * narrow experts exist; with 2 the narrow path's CUs also join that GEMM's
 * remaining tiles once both narrow GEMMs are done (a second launch of it on the
 * auxiliary stream), and the second wide GEMM waits for them.  Other values are
 * rejected.  Shapes with T*top_k <= 2*E*max_rows (small experts dominate) use
 * no auxiliary stream: each narrow GEMM runs on the caller's stream after the
 * wide one, on every CU (and wide_share does not apply).
 * It also stays off when H/128 or I/128 is odd or above 64, and for a first call made
 * while the caller's stream is being captured into a graph (the auxiliary
 * stream is created on the first call that is not captured).  Defaults come
 * from HKMOE_NARROW_CUS, HKMOE_NARROW_MAX and HKMOE_NARROW_SHARE in the
 * environment, else 64, 64 and 1 (out-of-range HKMOE_NARROW_SHARE is clamped to 0..2).  Concurrent hkmoe_moe_forward calls on one
 * device enqueue their fork/join one at a time (a mutex).
 * No reference counterpart: the reference has no grouped GEMM.
 */
int hkmoe_set_narrow(int32_t cus, int32_t max_rows, int32_t wide_share);
int hkmoe_get_narrow(int32_t* cus, int32_t* max_rows, int32_t* wide_share);

/*
 * Kernel timing of the layer entry points (measurement).  The reference times a
 * kernel with a hipEvent pair around its launch (kernels/cdna4/gemm/mxfp8/
 * MXFP8_4wave/4_wave.cu:517-571); here the events belong to the dispatches
 * themselves, so a layer call is timed per kernel without marker packets
 * between its kernels.
 *   hkmoe_kernel_timing(calls): calls > 0 times the kernels of the following
 *     hkmoe_moe_forward / hkmoe_moe_forward_mx / hkmoe_moe_forward_noalloc calls on
 *     the current device, cycling over `calls` sets of events (call i uses set
 *     i % calls, counting from this call); 0 turns it off.  Creates (and
 *     frees) events: not for use under graph capture.
 *   hkmoe_kernel_timing_read(set, begin_ms, end_ms, n): after the timed calls
 *     completed (the caller synchronises), the start and end of each role's
 *     kernel in ms from the start of the call's first kernel, or -1 for both
 *     when the call launched no kernel of that role; n >= HKMOE_TIMING_ROLES.
 */
#define HKMOE_TIMING_ROUTE 0          /* route_topk */
#define HKMOE_TIMING_BLOCK_SCAN 1     /* per-expert prefix over routing blocks */
#define HKMOE_TIMING_OFFSETS 2        /* expert offsets, M-tile list, counters */
#define HKMOE_TIMING_SCATTER 3        /* perm / inv_perm */
#define HKMOE_TIMING_MX_WORDS 4       /* MX layer: activation exponent words */
#define HKMOE_TIMING_GEMM1 5          /* grouped GEMM 1, 256x256 tiles */
#define HKMOE_TIMING_GEMM1_NARROW 6   /* grouped GEMM 1, narrow experts */
#define HKMOE_TIMING_GEMM1_JOIN 7     /* late-join launch of GEMM 1 (wide_share 2) */
#define HKMOE_TIMING_REQUANT 8        /* per-tensor requantisation of h */
#define HKMOE_TIMING_GEMM2 9          /* grouped GEMM 2, 256x256 tiles */
#define HKMOE_TIMING_GEMM2_NARROW 10  /* grouped GEMM 2, narrow experts */
#define HKMOE_TIMING_COMBINE 11       /* top-k weighted combine */
#define HKMOE_TIMING_ROLES 12
int hkmoe_kernel_timing(int32_t calls);
int hkmoe_kernel_timing_read(int32_t set, float* begin_ms, float* end_ms, int32_t n);
int hkmoe_moe_forward(const void* x_q, const float* x_scale, const float* logits, const void* w13,
                      const float* w13_scale, const void* w2, const float* w2_scale,
                      int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                      int32_t inter, int scale_mode, int w_layout, void* out, void* workspace,
                      size_t workspace_bytes, hkmoe_stream_t stream);

/*
 * hkmoe_moe_forward without a workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc.  No counterpart in the reference.
 *
 * Same arguments, results and errors as hkmoe_moe_forward (bit for bit), and it
 * allocates nothing: the layer's workspace is the library's per-device scratch
 * array of HKMOE_NOALLOC_SCRATCH_BYTES (64 MiB), which every GPU the library
 * runs on holds until the process ends.  A layer whose workspace
 * (hkmoe_moe_workspace_size) is larger is rejected with HKMOE_ERR_WORKSPACE
 * before any launch.  Largest T that fits: 509 for config-3 shapes (H=7168,
 * I=2048, E=256, top-8, block scales), 856 for config-5 shapes (H=4096, I=1536,
 * E=128, top-8), 655 for config-2 shapes (H=4096, I=14336, E=8, top-2,
 * per-tensor scales).  Every kernel runs on `stream`: the narrow path's auxiliary
 * stream is not used, so block-scaled layers with T*k <= 2*E*max_rows (see
 * hkmoe_set_narrow; every layer of the three shapes above that fits the scratch)
 * take the one-stream narrow schedule, as hkmoe_moe_forward does, and larger
 * ones run the 256x256 kernels alone.  The first call on a device looks up that device's scratch
 * address (hipGetSymbolAddress): make it outside graph capture.  All calls on
 * one device share its scratch and each call leaves its intermediates there:
 * calls that overlap in time on one device (other streams, other threads)
 * race and must be serialised by the caller.
 */
#define HKMOE_NOALLOC_SCRATCH_BYTES (64ull << 20)
int hkmoe_moe_forward_noalloc(const void* x_q, const float* x_scale, const float* logits, const void* w13,
                              const float* w13_scale, const void* w2, const float* w2_scale,
                              int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                              int32_t inter, int scale_mode, int w_layout, void* out, hkmoe_stream_t stream);

/*
 * Synthetic-input helpers (quantisers): x [R, C] fp32 on the device.
 *   hkmoe_quant_group:  q [R,C] e4m3, s [R, C/128]  (1x128 groups, row-major s)
 *   hkmoe_quant_block:  q [B,R,C] e4m3, s [B, R/128, C/128] (128x128 blocks)
 *   hkmoe_quant_tensor: q [R,C], s [1]; amax_ws: one fp32 of device scratch.
 * Scale = amax/448 (1.0 for an all-zero block); q = e4m3(x / s) RNE, saturating.
 * Bit-exact for finite x; a NaN gives +-448 (0x7E | sign), and block maxima
 * skip NaNs.
 */
int hkmoe_quant_group(const float* x, int64_t rows, int64_t cols, void* q, float* s,
                      hkmoe_stream_t stream);
int hkmoe_quant_block(const float* x, int64_t batch, int64_t rows, int64_t cols, void* q, float* s,
                      hkmoe_stream_t stream);
int hkmoe_quant_tensor(const float* x, int64_t rows, int64_t cols, void* q, float* s,
                       float* amax_ws, hkmoe_stream_t stream);

/*
 * MX (microscaling) FP8: e4m3 elements with one e8m0 exponent per row and
 * 32-element K block.  An e8m0 byte s stands for 2^(s - 127).
 *
 * hkmoe_quant_mx: x [R, C] fp32 (finite) -> q [R, C] e4m3, s [R, C/32] e8m0,
 *   s = clamp(floor(log2(amax32)) + 127, 0, 254) (0 for an all-zero block),
 *   q = e4m3(x * 2^(127 - s)), round to nearest even.  floor(log2) is exact
 *   (the biased exponent of amax).  C % 32 == 0.
 *   Replaces quantize_fp8_kernel and compute_e8m0_scale
 *   (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:296-321, 368-373).
 */
int hkmoe_quant_mx(const float* x, int64_t rows, int64_t cols, void* q, void* s,
                   hkmoe_stream_t stream);

/*
 * hkmoe_mx_pack_scales: e8m0 s [R, C/32] -> packed [C/128, R64] uint32 words,
 *   R64 = R rounded up to a multiple of 64, the operand order of the scaled
 *   MFMA: word (kt, p) holds in byte g the exponent of row 64*(p/64) + 16*g +
 *   p%16 for K block 4*kt + (p%64)/16 (0 for rows >= R).  C % 128 == 0.
 *   For R % 64 == 0 the words equal the reference's pack_scales_kernel
 *   followed by repack_scales_for_mfma_kernel (4_wave.cu:323-364), i.e. the
 *   words its device-side pack_scales builds
 *   (include/cdna4/ops/warp/register/tile/mma.cuh:253-270).
 */
int hkmoe_mx_pack_scales(const void* s, int64_t rows, int64_t cols, void* packed,
                         hkmoe_stream_t stream);

/*
 * hkmoe_gemm_mx: C[M,N] = sum over K blocks kb of
 *     2^(sa[m,kb] - 127) * 2^(sb[n,kb] - 127) * sum_{k in kb} A[m,k] * B[n,k]
 *   A [M,K] e4m3 with packed scales a_scale [K/128, M64]; B [N,K] e4m3 with
 *   packed scales b_scale [K/128, N] (hkmoe_mx_pack_scales); fp32 accumulate,
 *   C bf16 (RNE) or fp32.  K % 128 == 0, N % 256 == 0, M arbitrary.
 *   Replaces mxfp8_gemm_4wave_kernel (4_wave.cu:77-292), which is launched
 *   with the packed scales of prepare_mxfp8_data (4_wave.cu:377-448).
 */
int hkmoe_gemm_mx(const void* a, const void* a_scale, const void* b, const void* b_scale, void* c,
                  int64_t m, int64_t n, int64_t k, int out_dtype, hkmoe_stream_t stream);

/*
 * MX (1x32 e8m0) mixture-of-experts layer: the same routing, grouped GEMMs and
 * combine as hkmoe_moe_forward, with MX operands instead of fp32 scales.  The
 * exponents are applied inside the scaled MFMA, so the grouped GEMMs carry no
 * per-K-block rescale of their accumulators.  The reference applies MX scales
 * in its dense MXFP8 kernel only (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/
 * 4_wave.cu:77-292); these entry points have no counterpart there.
 *
 * Exponent word layouts (uint32, byte g of a word = one e8m0 exponent):
 *   tile-aligned activation words, [K/128][ws] with ws =
 *     hkmoe_mx_words_per_step(rows, E): M tile m (expert order, first row row0)
 *     owns words m*256 .. m*256+255; word m*256+q of K step kt holds in byte g
 *     the exponent of row row0 + 64*(q/64) + 16g + q%16 for K block
 *     4kt + (q%64)/16 (0 past the tile's rows).  Words past the last M tile
 *     are neither written nor read.
 *   weight words, per B tile: [E][N/256][K/128][256]; word p of (expert e, N
 *     tile nt, K step kt) holds in byte g the exponent of B-tile row
 *     R = 64*(p/64) + 16g + p%16 for K block 4kt + (p%64)/16, where B-tile row R
 *     is weight row nt*256 + R, or with gate_up = I the fused gate/up row
 *     nt*128 + 32*(R>>6) + (R&31) + ((R>>5)&1)*I.
 *
 * hkmoe_mx_words_per_step: ws for `rows` expert rows over E experts.
 * hkmoe_mx_pack_weight_scales: e8m0 [E, N, K/32] -> weight words (load time).
 * hkmoe_mx_gather_scales: e8m0 of x [x_rows, K/32] -> tile-aligned words of the
 *   expert-ordered rows (row p read from x row gather[p] / gather_div, or p).
 * hkmoe_grouped_gemm1_mx: as hkmoe_grouped_gemm1 (x read in place through
 *   gather), out_format HKMOE_BF16: h bf16 [rows, I]; HKMOE_E4M3: h e4m3 [rows, I]
 *   requantised per 1x32 block (the hkmoe_quant_mx rule applied to the bf16 h)
 *   and its tile-aligned words h_words [I/128][ws].
 * hkmoe_grouped_gemm2_mx: y bf16 [rows, H] from hq e4m3 + hq_words and w2.
 * hkmoe_moe_forward_mx: the whole layer; x_e8m0 [T, H/32] bytes (from
 *   hkmoe_quant_mx), weight words from hkmoe_mx_pack_weight_scales; workspace
 *   from hkmoe_moe_workspace_size(..., HKMOE_SCALE_MX).
 */
int64_t hkmoe_mx_words_per_step(int64_t rows, int32_t num_experts);
int hkmoe_mx_pack_weight_scales(const void* s, int64_t num_experts, int64_t n, int64_t k, int32_t gate_up,
                                void* words, hkmoe_stream_t stream);
int hkmoe_mx_gather_scales(const void* s, int64_t x_rows, int32_t k, const int32_t* gather,
                           int32_t gather_div, const int32_t* offsets, const int32_t* mtile_offsets,
                           int32_t num_experts, int64_t rows, void* words, hkmoe_stream_t stream);
int hkmoe_grouped_gemm1_mx(const void* x, const void* x_words, const int32_t* gather, int32_t gather_div,
                           int64_t x_rows, const void* w13, const void* w13_words, const int32_t* offsets,
                           const int32_t* mtile_offsets, const int32_t* mtile_list, int64_t rows,
                           int32_t num_experts, int32_t hidden, int32_t inter, int w_layout,
                           int out_format, void* h, void* h_words, int32_t* tile_counters,
                           hkmoe_stream_t stream);
int hkmoe_grouped_gemm2_mx(const void* hq, const void* hq_words, const void* w2, const void* w2_words,
                           const int32_t* offsets, const int32_t* mtile_offsets,
                           const int32_t* mtile_list, int64_t rows, int32_t num_experts,
                           int32_t hidden, int32_t inter, int w_layout, void* y,
                           int32_t* tile_counters, hkmoe_stream_t stream);
int hkmoe_moe_forward_mx(const void* x_q, const void* x_e8m0, const float* logits, const void* w13,
                         const void* w13_words, const void* w2, const void* w2_words,
                         int64_t num_tokens, int32_t num_experts, int32_t top_k, int32_t hidden,
                         int32_t inter, int w_layout, void* out, void* workspace,
                         size_t workspace_bytes, hkmoe_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HKMOE_H */
