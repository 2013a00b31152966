// Persistent FP8 (e4m3 x e4m3 -> fp32) GEMM core for gfx950, shared by the
// dense GEMM and both grouped (per-expert) MoE GEMMs.
//
// C[m, n] = sum_k A[m, k] * B[n, k]   ("TN": both operands K-contiguous), the
// convention of the reference's mma_ABt kernels
// (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:77-292, cdna3
// 256_256_64_32.cpp:32-200).  Design (all new, CDNA4-first):
//
//  * block tile 256 (rows of A) x 256 (rows of B) x 128 (K), 8 waves as 2 x 4;
//    each wave owns a 128 x 64 sub-tile = 8 x 4 v_mfma_f32_16x16x128_f8f6f4.
//  * two LDS stages of 64 KiB (+1 KiB of activation scales) filled by
//    buffer_load_dwordx4 ... lds (no VGPR staging): 128-byte row segments, i.e.
//    whole L2 lines per lane octet.
//  * ping-pong: each K step is four barrier-separated phases per wave:
//    memory (LDS fragment reads + DMA issue), compute (MFMAs from registers
//    only, raised wave priority), memory, compute.  Waves 4-7 (rows 128-255)
//    run one phase behind waves 0-3, and each group passes one extra barrier
//    at opposite ends of the K loop, so on every SIMD one wave issues MFMAs
//    while the other reads LDS and issues loads.  Each group DMAs its own A
//    half one step ahead and half of B two steps ahead (a stage's B half is
//    free once both groups have read their B fragments, two phases before
//    its A half); every wave waits for its own DMA (vmcnt) and LDS reads
//    (lgkmcnt) before a barrier, which is what makes a stage visible / free
//    for the others.
//  * 16-byte chunk c of LDS row r is stored at c ^ ((r & 7) ^ ((r >> 3) & 1)):
//    the ds_read_b128 operand reads of 16 consecutive rows are bank-conflict
//    free whether the LDS serves 8 or 16 lanes per cycle, and the XOR is a lane
//    constant for every fragment; the swizzle is applied on the global side
//    because the DMA writes lanes linearly.
//  * 128x128 weight / 1x128 activation block scales: K step == scale block ==
//    the K extent of one v_mfma_f32_16x16x128, so every MFMA of a step starts
//    from zero and yields the block's raw product P_k, which is folded in as
//        C = fma(P_k, s_a[row, k] * s_w[col block, k], C)
//    (4 FMAs per MFMA, issued under the next MFMA).  C is in true units at
//    every step: no division by a scale, so no overflow when a block's scale
//    is tiny next to the previous one's, and no final rescale.
//  * MX (OCP microscaling) mode: 1x32 e8m0 exponents per row of A and of B,
//    applied inside the MFMA (v_mfma_scale_f32_16x16x128_f8f6f4), which takes
//    the exponent of row l%16 and K block l/16 from lane l: one e8m0 byte per
//    lane and operand, picked from a 32-bit word by the instruction's op_sel
//    (fragments are read in the instruction's K order, read_frag_mx).  The
//    scales arrive pre-packed so that word (k step kt, position p) of a 64-row
//    group holds, in byte g, the exponent of row 16g + p%16 of the group for K
//    block 4kt + (p%64)/16 (mx_pack_scales_kernel).  A tile's words of one K
//    step are then 1 KiB contiguous per operand, DMA'd by two instructions with
//    group 0's A half (2 KiB more per stage), and a lane reads one dword per
//    64-row group: no VALU rescale.
//  * optional row gather: A row of output row p is a_gather[p] / gather_div
//    (the expert-sorted permutation), so GEMM 1 reads token rows in place.
//  * MFMA operands are swapped (B fragment as src0) so each lane owns 4
//    consecutive columns of one output row per 16-row sub-tile: one activation
//    scale per lane per sub-tile and block.
//  * persistent grid (one 512-thread workgroup per CU).  Tiles form blocks of
//    bm x bn = 32 tiles (dense 4 x 8, grouped 2 x 16: a grouped block mostly
//    spans one or two experts, whose 16 N tiles then share the A rows).  The
//    grouped GEMMs walk M tiles in the order of an optional device list (full
//    tiles first, so blocks hold tiles of equal cost).  With tile counters
//    (grouped GEMMs) every XCD (one
//    L2; workgroups are dispatched round-robin, so blockIdx % 8) owns the
//    blocks b = x, x+8, ... and its 32 workgroups pull tiles of those blocks in
//    order from the XCD's atomic counter, so they keep working on the same
//    block and share its operand panels in L2 even when tiles differ in cost
//    (ragged experts); a drained queue steals from the other XCDs' queues.
//    Without counters (dense GEMM, equal tiles) the same blocks are walked
//    statically.
//  * ragged expert segments: the M-tile list comes from a device-side
//    mtile_offsets[E+1]; 16-row sub-tiles with no valid row skip their MFMAs.
//  * fused epilogues, staged through LDS and written as whole rows: bf16 store,
//    fp32 store, or SiLU(gate)*up with either a bf16 store + running |h| max
//    (per-tensor requantisation follows) or an in-tile 1x128-group
//    requantisation to e4m3 + scales (block mode).
#pragma once

#include "common.hpp"

namespace hkmoe {

enum class Epi : int { kStoreBf16 = 0, kStoreF32 = 1, kSiluBf16 = 2, kSiluQuant = 3, kSiluMx = 4 };
enum class Scale : int { kTensor = 0, kBlock = 1, kMX = 2 };

struct GemmParams {
  const uint8_t* a;            // A rows [a_rows, K] e4m3
  const int32_t* a_gather;     // optional: A row of output row p = a_gather[p] / gather_div
  const uint8_t* b;            // [E, nb, K] e4m3, row-major or packed (b_packed)
  void* c;                     // [rows, n_out]: bf16, fp32 or (kSiluQuant, kSiluMx) e4m3
  const float* a_scale;        // kTensor: [1] or null (1.0); kBlock: a_scale[r*as_rs + kb*as_ks]
                               // kMX: packed e8m0 words [K/128][as_rs]; dense: by row (as_rs =
                               // rows rounded up to 64); grouped: by M tile m, words m*256 ..
  const float* b_scale;        // kTensor: [E] or null (1.0); kBlock: [E, nb/128, K/128]
                               // kMX: packed e8m0 words; dense [K/128][nb]; grouped, per
                               // B tile: [E][nb/256][K/128][256] (word p = B tile row p)
  float* c_scale;              // kSiluQuant: group scales, transposed [n_out/128, rows]
                               // kSiluMx: packed e8m0 words of h, [n_out/128][cs_rs] by M tile
  const int32_t* offsets;      // [E+1] row offsets; nullptr = dense (one segment of `rows`)
  const int32_t* mtile_offsets;// [E+1] M-tile offsets; nullptr = dense
  const int32_t* mtile_list;   // optional [M tiles][2] = (expert, first row), in schedule order
  float* amax;                 // kSiluBf16: running max |h| (uint-ordered), may be null
  int32_t* tile_ctr;           // optional: 8 zeroed per-XCD tile counters (dynamic schedule)
                               // (narrow kernel: zeroed item counter at [0], active-slot
                               // counter at [2])
  const int32_t* narrow_cnt;   // optional: the last *narrow_cnt M-tile list entries belong to
                               // the narrow kernel (gemm_narrow.hpp); this kernel skips them
  int32_t yield_from;          // > 0: with narrow tiles present, workgroups >= yield_from exit
                               // at once (their CUs go to the narrow kernel);
                               // < 0: a second launch that joins the tile queues once the
                               // narrow kernels are done; it exits at once without narrow tiles
  int32_t narrow_active;       // narrow kernel: workgroups that take items while 256x256
                               // tiles exist (0: all); without such tiles, all of them do
  int64_t rows;                // output rows (dense: M)
  int64_t a_rows;              // rows addressable through `a`
  int64_t as_rs, as_ks;        // activation scale strides (row, K block)
  uint32_t a_bytes;            // buffer bound of `a`: min(a_rows * K, 2^32 - 1)
  int32_t gather_div;
  int32_t num_experts;
  int32_t K;
  int32_t nb;                  // B rows per expert (N, or 2I for the fused gate/up GEMM)
  int32_t n_out;               // output columns (N, or I)
  int32_t n_tiles;             // N tiles per M tile
  int32_t b_packed;            // 1: b is in the packed tile layout of pack_weights_kernel
  int32_t blk_m_log2;          // tile blocks are 2^blk_m_log2 M tiles x 32 / 2^blk_m_log2 N tiles
  int64_t cs_rs;               // kSiluMx: words per K step of the packed h exponents
};

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = kBM * kBK;                    // 32 KiB per operand per stage
constexpr int kScaleBytes = kBM * 4;                     // activation scales of one K block
constexpr int kStageBytes = 2 * kTileBytes + kScaleBytes;
constexpr int kMaxKBlocks = 128;                         // K <= 16384
constexpr int kBsBytes = 2 * kMaxKBlocks * 4;            // weight scales of one tile
constexpr int kMainLds = 2 * kStageBytes + kBsBytes;
// epilogue staging of a bf16 output tile, rows padded by 16 bytes
constexpr int kCtLdStore = kBN + 8;                      // bf16 elements per staged row
constexpr int kCtLdSilu = 128 + 8;
constexpr int kEpiLds = kBM * kCtLdStore * 2;
static_assert(kBM * kCtLdSilu * 2 + kBM * 4 <= kEpiLds, "SiLU staging + MX exponents fit the epilogue LDS");
constexpr int kLdsData = kMainLds > kEpiLds ? kMainLds : kEpiLds;
constexpr int kLdsBytes = kLdsData + 16;                 // + the broadcast slot of the tile queue
constexpr int kGroupM = 8;

static_assert(kLdsBytes <= 160 * 1024, "LDS budget");

// XOR applied to the 16-byte chunk index of 128-byte LDS row r.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// One 16x128 operand fragment (32 bytes per lane: row l % 16, K bytes
// 32*(l/16) .. +31) from a swizzled 128-byte-row tile; `x` = swz(row).
__device__ __forceinline__ i32x8 read_frag(const uint8_t* tile, int row, int half, int x) {
  const uint8_t* base = tile + row * kBK;
  const i32x4 lo = *reinterpret_cast<const i32x4*>(base + ((2 * half) ^ x) * 16);
  const i32x4 hi = *reinterpret_cast<const i32x4*>(base + ((2 * half + 1) ^ x) * 16);
  i32x8 r;
  r.s0 = lo.x; r.s1 = lo.y; r.s2 = lo.z; r.s3 = lo.w;
  r.s4 = hi.x; r.s5 = hi.y; r.s6 = hi.z; r.s7 = hi.w;
  return r;
}

// The same fragment in the scaled MFMA's K order, which the e8m0 scales need
// (the unscaled instruction accepts any common order of both operands): lane
// l holds K bytes 16g .. 16g+15 in registers 0-3 and 64+16g .. 64+16g+15 in
// registers 4-7 (g = l/16), so 32-byte K block b lies in lane groups 2(b%2)
// and 2(b%2)+1, and the instruction takes block b's exponent for row l%16 from
// lane group b.
__device__ __forceinline__ i32x8 read_frag_mx(const uint8_t* tile, int row, int lg, int x) {
  const uint8_t* base = tile + row * kBK;
  const i32x4 lo = *reinterpret_cast<const i32x4*>(base + (lg ^ x) * 16);
  const i32x4 hi = *reinterpret_cast<const i32x4*>(base + ((lg + 4) ^ x) * 16);
  i32x8 r;
  r.s0 = lo.x; r.s1 = lo.y; r.s2 = lo.z; r.s3 = lo.w;
  r.s4 = hi.x; r.s5 = hi.y; r.s6 = hi.z; r.s7 = hi.w;
  return r;
}

template <bool MX>
__device__ __forceinline__ i32x8 read_operand(const uint8_t* tile, int row, int lg, int x) {
  if constexpr (MX) return read_frag_mx(tile, row, lg, x);
  else return read_frag(tile, row, lg, x);
}

// silu(g) = g / (1 + e^-g) with the hardware exp2 and reciprocal (a few ulp;
// the result is rounded to bf16 next).
__device__ __forceinline__ float silu(float g) {
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * 1.4426950408889634f));
}

// Tile row of activation-scale slot s: the lane with l16 = r % 16 of wave-row
// r / 128 reads its 8 sub-tile scales as 8 consecutive floats.
__device__ __forceinline__ int scale_slot_row(int slot) {
  const int wm = slot >> 7, w = slot & 127;
  return wm * 128 + (w & 7) * 16 + (w >> 3);
}

// Scaled MFMA with e8m0 operand scales: byte OPB of sb scales the B fragment
// (src0), byte OPA of sa the A fragment (src1); e4m3 operands.
template <int OPB, int OPA>
__device__ __forceinline__ f32x4 mfma_mx(const i32x8& b, const i32x8& a, f32x4 c, int sb, int sa) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(b, a, c, 0, 0, OPB, sb, OPA, sa);
}

// One A sub-tile (16 rows, exponent byte U of sa) against the wave's four B
// fragments (exponent bytes 0-3 of sb).
template <int U>
__device__ __forceinline__ void mx_subtile(f32x4 (&acc)[4], const i32x8 (&bf)[4], const i32x8& af,
                                           int sb, int sa) {
  acc[0] = mfma_mx<0, U>(bf[0], af, acc[0], sb, sa);
  acc[1] = mfma_mx<1, U>(bf[1], af, acc[1], sb, sa);
  acc[2] = mfma_mx<2, U>(bf[2], af, acc[2], sb, sa);
  acc[3] = mfma_mx<3, U>(bf[3], af, acc[3], sb, sa);
}

// Block scales: c += f * p element-wise, one fused multiply-add each (p: one
// K block's raw MFMA product, f: its scale product).  The 256x256 and the
// narrow kernel both fold through here, so they give the same bits.
__device__ __forceinline__ void fold_block(f32x4& c, const f32x4& p, float f) {
  c[0] = __builtin_fmaf(p[0], f, c[0]);
  c[1] = __builtin_fmaf(p[1], f, c[1]);
  c[2] = __builtin_fmaf(p[2], f, c[2]);
  c[3] = __builtin_fmaf(p[3], f, c[3]);
}

// Wait for this wave's outstanding DMA and LDS reads, then the workgroup
// barrier; the asm memory clobber keeps the compiler from moving memory
// operations across it.
__device__ __forceinline__ void sync_stage() {
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
__device__ __forceinline__ void sync_lds() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <Epi EPI, Scale SC>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_persistent(GemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  float* bs_lds = reinterpret_cast<float*>(smem + 2 * kStageBytes);  // [2][k_blocks]

  constexpr bool kBlockSc = (SC == Scale::kBlock);
  constexpr bool kMX = (SC == Scale::kMX);
  constexpr bool kSilu = (EPI == Epi::kSiluBf16 || EPI == Epi::kSiluQuant || EPI == Epi::kSiluMx);
  // stage: A tile, B tile, A scales (1 KiB) and, in MX mode, B scales (1 KiB)
  constexpr int kStg = kMX ? kStageBytes + kScaleBytes : kStageBytes;
  static_assert(EPI != Epi::kSiluMx || kMX, "MX requantisation needs MX scales");
  static_assert(2 * kStg <= kLdsData, "LDS budget");

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int grp = wave >> 2;  // ping-pong group == 128-row half of the tile
  const int wg = wave & 3;    // wave within the group == 64-column quarter
  const int l16 = lane & 15;
  const int lg = lane >> 4;   // 0..3
  const int wave_row0 = grp * 128;
  const int fx = swz(l16);    // fragment rows are l16 + multiples of 16

  // leave this CU to the narrow kernel when it has work (device-side decision:
  // the host does not know the expert sizes)
  if (p.narrow_cnt != nullptr && p.yield_from != 0) {
    const int ncnt = __builtin_amdgcn_readfirstlane(*p.narrow_cnt);
    if (p.yield_from > 0 ? (ncnt > 0 && static_cast<int>(blockIdx.x) >= p.yield_from) : ncnt == 0) return;
  }
  const bool dense = (p.offsets == nullptr);
  const int total_mtiles = dense ? static_cast<int>((p.rows + kBM - 1) / kBM)
                                 : __builtin_amdgcn_readfirstlane(p.mtile_offsets[p.num_experts] -
                                                                  (p.narrow_cnt ? *p.narrow_cnt : 0));
  const int k_steps = p.K / kBK;

  // XCD-aware virtual id: workgroups are dispatched round-robin over 8 XCDs,
  // so blockIdx % 8 is the XCD; give each XCD a contiguous run of ids.
  const int g = gridDim.x;
  const int vid = (g & 7) == 0 ? (blockIdx.x & 7) * (g >> 3) + (blockIdx.x >> 3) : blockIdx.x;

  // DMA geometry: wave instruction i of wave wg (in its group) fills 8 LDS rows
  // 32*i + 8*wg + lane/8 (+ the group's half for A); the lane fetches logical
  // chunk (lane & 7) ^ swz(row), which lands swizzled.  swz does not depend on i.
  const int ld_row = 8 * wg + (lane >> 3);
  const int ld_chunk = (lane & 7) ^ swz(ld_row);
  const i32x4 a_srd = make_srd(p.a, p.a_bytes);

  // tile blocks: bm M tiles x bn N tiles, bm * bn = 32
  const int bm = 1 << p.blk_m_log2, bn = 32 >> p.blk_m_log2;
  const int nbn = (p.n_tiles + bn - 1) / bn;
  const int nblocks = ((total_mtiles + bm - 1) / bm) * nbn;
  int* s_tile = reinterpret_cast<int*>(smem + kLdsData);
  const int xcd = blockIdx.x & 7;
  int steal = 0;          // queues visited so far (thread 0 only)
  int static_j = vid;     // static schedule: next slot index

  while (true) {
    // ---- next tile: slot j of queue q -> block b = q + 8*(j/32) -----------
    int mt_glob = -1, nt = 0;
    if (p.tile_ctr != nullptr) {
      if (tid == 0) {
        int t = -1;
        while (steal < 8 && t < 0) {
          const int q = (xcd + steal) & 7;
          const int nslots = q < nblocks ? 32 * ((nblocks - q + 7) >> 3) : 0;
          const int j = nslots > 0 ? atomicAdd(&p.tile_ctr[q], 1) : nslots;
          if (j >= nslots) { ++steal; continue; }
          const int b = q + 8 * (j >> 5), sl = j & 31;
          const int m = bm * (b / nbn) + (sl & (bm - 1)), n = bn * (b % nbn) + (sl >> p.blk_m_log2);
          if (m < total_mtiles && n < p.n_tiles) t = m * p.n_tiles + n;
        }
        *s_tile = t;
      }
      __syncthreads();
      const int t = *s_tile;
      if (t < 0) break;
      mt_glob = t / p.n_tiles;
      nt = t - mt_glob * p.n_tiles;
    } else {
      // same blocks, walked statically: vid-th slot of every round of g slots
      bool found = false;
      while (!found) {
        const int j = static_j;
        static_j += g;
        const int b = j >> 5, sl = j & 31;
        if (b >= nblocks) break;
        const int m = bm * (b / nbn) + (sl & (bm - 1)), n = bn * (b % nbn) + (sl >> p.blk_m_log2);
        if (m < total_mtiles && n < p.n_tiles) { mt_glob = m; nt = n; found = true; }
      }
      if (!found) break;
    }
    mt_glob = __builtin_amdgcn_readfirstlane(mt_glob);
    nt = __builtin_amdgcn_readfirstlane(nt);

    // ---- M tile -> expert segment ----------------------------------------
    int e = 0, row0 = 0, valid = 0;
    int mnat = mt_glob;  // M tile index in expert order (MX exponent words are by M tile)
    if (dense) {
      row0 = mt_glob * kBM;
      valid = static_cast<int>(min<int64_t>(kBM, p.rows - row0));
    } else if (p.mtile_list != nullptr) {
      e = p.mtile_list[2 * mt_glob];
      row0 = p.mtile_list[2 * mt_glob + 1];
      valid = min(kBM, p.offsets[e + 1] - row0);
      mnat = p.mtile_offsets[e] + (row0 - p.offsets[e]) / kBM;
    } else {
      int lo = 0, hi = p.num_experts;  // largest e with mtile_offsets[e] <= mt_glob
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (p.mtile_offsets[mid] <= mt_glob) lo = mid; else hi = mid;
      }
      e = lo;
      row0 = p.offsets[e] + (mt_glob - p.mtile_offsets[e]) * kBM;
      valid = min(kBM, p.offsets[e + 1] - row0);
    }
    e = __builtin_amdgcn_readfirstlane(e);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    mnat = __builtin_amdgcn_readfirstlane(mnat);
    valid = __builtin_amdgcn_readfirstlane(valid);

    // B (group 0 only): LDS row 32*i + ld_row holds weight row b_row0 + boff(i)
    //   plain: nt*256 + r                       -> boff(i) = 32*i
    //   SiLU:  quarter q = r >> 6 = i >> 1 holds 32 gate rows (i even) then
    //          the 32 matching up rows (i odd) -> boff(i) = 32*(i>>1) + (i&1)*I
    // Row-major weights: lane offset of that row and chunk, K step kt at byte
    // kt*128.  Packed weights: the tile's K step kt is the 32 KiB stage image
    // at kt*32 KiB of the tile's own panel, so instruction i of wave wg reads
    // the 1 KiB at (32*i + 8*wg)*128 linearly.
    // Lane offsets of the two register halves of a B fragment within its
    // 2 KiB of the stage: fragment-major (packed weights) or swizzled rows,
    // in the K order of the MFMA variant (read_frag / read_frag_mx).
    int b_lo, b_hi;
    if (p.b_packed) {
      if constexpr (kMX) {
        b_lo = (lg & 1) * 1024 + ((lg >> 1) * 16 + l16) * 16;
        b_hi = (lg & 1) * 1024 + (((lg >> 1) + 2) * 16 + l16) * 16;
      } else {
        b_lo = lane * 16;
        b_hi = 1024 + lane * 16;
      }
    } else {
      b_lo = l16 * kBK + ((kMX ? lg : 2 * lg) ^ fx) * 16;
      b_hi = l16 * kBK + ((kMX ? lg + 4 : 2 * lg + 1) ^ fx) * 16;
    }
    i32x4 b_srd;
    int b_voff, b_kstride;
    if (p.b_packed) {
      b_srd = make_srd(p.b + (static_cast<int64_t>(e) * (p.nb / kBN) + nt) * kBN * p.K,
                       static_cast<uint32_t>(kBN) * p.K);
      b_voff = wg * 8 * kBK + lane * 16;
      b_kstride = kTileBytes;
    } else {
      b_srd = make_srd(p.b + static_cast<int64_t>(e) * p.nb * p.K, static_cast<uint32_t>(p.nb) * p.K);
      const int b_row0 = kSilu ? nt * 128 + ld_row : nt * kBN + ld_row;
      b_voff = b_row0 * p.K + ld_chunk * 16;
      b_kstride = kBK;
    }

    // A (own half): LDS row grp*128 + 32*i + ld_row <- A row of output row
    // row0 + min(r, valid - 1); 16-row sub-tiles past `valid` are not loaded.
    int a_voff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = row0 + min(wave_row0 + 32 * i + ld_row, valid - 1);
      const int ar = p.a_gather ? p.a_gather[rr] / p.gather_div : rr;
      a_voff[i] = ar * p.K + ld_chunk * 16;
    }
    // activation scales of the own half: waves 0,1 of each group gather 64 slots
    const bool scale_loader = kBlockSc && wg < 2;
    int as_voff = 0;
    if (scale_loader) {
      const int rr = row0 + min(scale_slot_row(wave_row0 + wg * 64 + lane), valid - 1);
      const int ar = p.a_gather ? p.a_gather[rr] / p.gather_div : rr;
      as_voff = static_cast<int>(ar * p.as_rs) * 4;
    }
    // MX: a tile's exponent words of one K step are 1 KiB contiguous per
    // operand, so wave 0 DMAs all 256 A words and wave 1 all 256 B words (one
    // 16-byte-per-lane instruction each), with group 0's A half.  Group 1 last
    // read that stage's words three phases earlier (its first memory phase of
    // the step before).  Words past the packed arrays read as zero (rows that
    // are never stored).
    const bool mx_loader = kMX && wave < 2;
    i32x4 mx_srd;
    int mx_voff = 0, mx_kstride = 0, mx_lds = 0;
    if constexpr (kMX) {
      const int k_steps_ = p.K / kBK;
      if (wave == 0) {
        mx_srd = make_srd(p.a_scale, static_cast<uint32_t>(k_steps_ * p.as_rs * 4));
        mx_voff = (mnat * kBM + lane * 4) * 4;
        mx_kstride = static_cast<int>(p.as_rs) * 4;
        mx_lds = 2 * kTileBytes;
      } else if (dense) {
        mx_srd = make_srd(p.b_scale, static_cast<uint32_t>(k_steps_ * p.nb * 4));
        mx_voff = (nt * kBN + lane * 4) * 4;
        mx_kstride = p.nb * 4;
        mx_lds = 2 * kTileBytes + kScaleBytes;
      } else {
        // this B tile's words: k_steps_ consecutive KiB
        const int ntiles = p.nb / kBN;
        mx_srd = make_srd(reinterpret_cast<const uint8_t*>(p.b_scale) +
                              (static_cast<int64_t>(e) * ntiles + nt) * k_steps_ * 1024,
                          static_cast<uint32_t>(k_steps_) * 1024);
        mx_voff = lane * 16;
        mx_kstride = 1024;
        mx_lds = 2 * kTileBytes + kScaleBytes;
      }
    }

    // DMA instructions of one K step issued by this wave.  issue_a: its
    // group's A half (4, dead 16-row sub-tiles skipped) and, for waves 0-1 of
    // each group, the activation scales (1).  issue_b: exactly 4 loads, half
    // of the B stage (group 0 rows 0-127, group 1 rows 128-255); being the
    // last 4 loads a wave issues, they are what vmcnt(4) leaves in flight.
    auto issue_a = [&](int kt) {
      uint8_t* sa = smem + (kt & 1) * kStg;
      const int koff = kt * kBK;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r8 = wave_row0 + 32 * q + 8 * wg;  // first row of this wave load
        if ((r8 & ~15) < valid) load_lds_16B(a_srd, sa + r8 * kBK, a_voff[q], koff);
      }
      if (scale_loader) {
        const i32x4 as_srd = make_srd(p.a_scale, 0xffffffffu);
        load_lds_4B(as_srd, sa + 2 * kTileBytes + (wave_row0 + wg * 64) * 4, as_voff,
                    static_cast<int>(kt * p.as_ks) * 4);
      }
      if (mx_loader) load_lds_16B(mx_srd, sa + mx_lds, mx_voff, kt * mx_kstride);
    };
    auto issue_b = [&](int kt) {
      uint8_t* sb = smem + (kt & 1) * kStg + kTileBytes;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int i = grp * 4 + q;
        const int boff = kSilu ? (32 * (i >> 1) + ((i & 1) ? p.n_out : 0)) : 32 * i;
        const int ioff = p.b_packed ? 32 * i * kBK : boff * p.K;
        load_lds_16B(b_srd, sb + (32 * i + 8 * wg) * kBK, b_voff, kt * b_kstride + ioff);
      }
    };
    // every load of this wave except its last issue_b has completed
    auto wait_dma = [&](bool b_in_flight) {
      if (b_in_flight) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int live_sub = max(0, min(8, (valid - wave_row0 + 15) >> 4));

    __syncthreads();  // previous tile is done with every LDS buffer
    if constexpr (kBlockSc) {
      // weight scales of this tile for every K block: [2][k_steps]
      const float* bs = p.b_scale + static_cast<int64_t>(e) * (p.nb / kGroup) * k_steps;
      const int nb0 = kSilu ? nt : 2 * nt;                           // gate / first n block
      const int nb1 = kSilu ? (p.n_out / kGroup + nt) : 2 * nt + 1;  // up / second n block
      for (int t = tid; t < 2 * k_steps; t += kThreads) {
        const int h = t >= k_steps;
        bs_lds[t] = bs[(h ? nb1 : nb0) * k_steps + (t - h * k_steps)];
      }
    }
    issue_a(0);
    issue_b(0);
    if (k_steps > 1) issue_b(1);
    wait_dma(k_steps > 1);     // stage 0 (and the weight scales) visible to all
    if (grp == 1) sync_lds();  // group 1 runs one phase behind group 0

    // block scales of the current K step: the activation scale of each of the
    // lane's 8 sub-tile rows, and the weight scale of its gate / up (or only)
    // 128-column block
    float sa_cur[8], sb_cur0 = 1.0f, sb_cur1 = 1.0f;

    // Four barrier-separated phases per K step: memory (LDS fragment reads,
    // DMA issue), compute (MFMAs from registers only), memory, compute.  Group
    // 1 is one phase behind, so on every SIMD one wave issues MFMAs while the
    // other reads LDS.  Phase p of the block is group 0's phase p and group
    // 1's phase p-1.  Stage kt is read in phases 4kt..4kt+3, its B fragments
    // only in 4kt and 4kt+1: so A(kt+1) is issued in the first memory phase
    // of step kt (phases 4kt / 4kt+1) and B(kt+2), into the B half of stage
    // kt, in the second (phases 4kt+2 / 4kt+3), more than a step ahead.
    // Stage kt+1 is first read in phase 4kt+4: every wave waits for all its
    // loads but the newest B(kt+2) before the barrier ending phase 4kt+3
    // (group 0: end of its second compute phase; group 1: end of its second
    // memory phase).
    for (int kt = 0; kt < k_steps; ++kt) {
      const bool more = kt + 1 < k_steps;
      const uint8_t* sa = smem + (kt & 1) * kStg;
      const uint8_t* sb = sa + kTileBytes;

      // ---- memory phase 1: B fragments, A sub-tiles 0-3, scales, DMA kt+1
      i32x8 bf[4], af[4];
      int mx_sb = 0, mx_sa0 = 0, mx_sa1 = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint8_t* fb = sb + (wg * 4 + j) * 2048;
        const i32x4 lo = *reinterpret_cast<const i32x4*>(fb + b_lo);
        const i32x4 hi = *reinterpret_cast<const i32x4*>(fb + b_hi);
        bf[j].s0 = lo.x; bf[j].s1 = lo.y; bf[j].s2 = lo.z; bf[j].s3 = lo.w;
        bf[j].s4 = hi.x; bf[j].s5 = hi.y; bf[j].s6 = hi.z; bf[j].s7 = hi.w;
      }
      if constexpr (kMX) {
        // exponent words: B rows wg*64 + 16j + l16 (byte j), A rows of
        // sub-tiles 0-3 and 4-7 (byte i % 4), all for K block 4kt + lg
        const int* sw = reinterpret_cast<const int*>(sb + kTileBytes);
        mx_sa0 = sw[wave_row0 + lane];
        mx_sa1 = sw[wave_row0 + 64 + lane];
        mx_sb = sw[kBM + wg * 64 + lane];
      }
      if (live_sub > 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = read_operand<kMX>(sa, wave_row0 + i * 16 + l16, lg, fx);
      }
      if constexpr (kBlockSc) {
        // this step's scales; the factors are formed in the compute phases
        const float* sc = reinterpret_cast<const float*>(sb + kTileBytes) + wave_row0 + l16 * 8;
        const f32x4 s_lo = *reinterpret_cast<const f32x4*>(sc);
        const f32x4 s_hi = *reinterpret_cast<const f32x4*>(sc + 4);
        sa_cur[0] = s_lo.x; sa_cur[1] = s_lo.y; sa_cur[2] = s_lo.z; sa_cur[3] = s_lo.w;
        sa_cur[4] = s_hi.x; sa_cur[5] = s_hi.y; sa_cur[6] = s_hi.z; sa_cur[7] = s_hi.w;
        if constexpr (kSilu) {
          sb_cur0 = bs_lds[kt];
          sb_cur1 = bs_lds[k_steps + kt];
        } else {
          sb_cur0 = sb_cur1 = bs_lds[(wg >> 1) * k_steps + kt];
        }
      }
      if (more) issue_a(kt + 1);
      sync_lds();
      __builtin_amdgcn_sched_barrier(0);

      // ---- compute phase 1: sub-tiles 0-3
      auto compute = [&](int i0) {
        __builtin_amdgcn_s_setprio(1);
        // Skipped only when all four sub-tiles are dead; a partly live phase
        // also computes its dead sub-tiles (stale fragments, never stored).
        if (live_sub > i0) {
          if constexpr (kMX) {
            const int sa_w = i0 == 0 ? mx_sa0 : mx_sa1;
            mx_subtile<0>(acc[i0 + 0], bf, af[0], mx_sb, sa_w);
            mx_subtile<1>(acc[i0 + 1], bf, af[1], mx_sb, sa_w);
            mx_subtile<2>(acc[i0 + 2], bf, af[2], mx_sb, sa_w);
            mx_subtile<3>(acc[i0 + 3], bf, af[3], mx_sb, sa_w);
          } else if constexpr (kBlockSc) {
            // factor of sub-tile u: its row's activation scale times the
            // weight scale of the column block (gate: j < 2, up: j >= 2)
            float f0[4], f1[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              f0[u] = sa_cur[i0 + u] * sb_cur0;
              f1[u] = kSilu ? sa_cur[i0 + u] * sb_cur1 : f0[u];
            }
            // MFMA t from zero; the FMAs of MFMA t-1 follow it, so they run
            // while MFMA t occupies the matrix core
            f32x4 prev = mfma_e4m3_16x16x128(bf[0], af[0], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int t = 1; t <= 16; ++t) {
              f32x4 cur;
              if (t < 16) cur = mfma_e4m3_16x16x128(bf[t & 3], af[t >> 2], f32x4{0.f, 0.f, 0.f, 0.f});
              const int u = (t - 1) >> 2, j = (t - 1) & 3;
              fold_block(acc[i0 + u][j], prev, (kSilu && j >= 2) ? f1[u] : f0[u]);
              if (t < 16) prev = cur;
            }
          } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
              const int u = t >> 2, j = t & 3;
              acc[i0 + u][j] = mfma_e4m3_16x16x128(bf[j], af[u], acc[i0 + u][j]);
            }
          }
        }
        __builtin_amdgcn_s_setprio(0);
      };
      compute(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);

      // ---- memory phase 2: A sub-tiles 4-7
      if (live_sub > 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = read_operand<kMX>(sa, wave_row0 + (i + 4) * 16 + l16, lg, fx);
      }
      const bool more2 = kt + 2 < k_steps;
      if (more2) issue_b(kt + 2);
      if (grp == 1) wait_dma(more2); else sync_lds();
      __builtin_amdgcn_sched_barrier(0);

      // ---- compute phase 2: sub-tiles 4-7
      compute(4);
      __builtin_amdgcn_sched_barrier(0);
      if (grp == 0) wait_dma(more2); else __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
    }
    if (grp == 0) sync_lds();  // group 0's extra barrier pairs with group 1's first

    // ---- epilogue ----------------------------------------------------------
    // lane holds, for sub-tile i and n fragment j, output row wave_row0+16i+l16
    // and columns 16*j + 4*lg .. +3 of the wave's 64-column quarter
    // per-tensor scales are applied here; block-scaled and MX accumulators
    // already hold the scaled sums
    float tens = 1.0f;
    if constexpr (SC == Scale::kTensor)
      tens = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[e] : 1.0f);
    auto fac = [&](int, int) -> float { return tens; };

    if constexpr (EPI == Epi::kStoreF32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave_row0 + i * 16 + l16;
        if (i < live_sub && r < valid) {
          const float f = fac(i, 0);
          float* crow = static_cast<float*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out + nt * kBN + wg * 64;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 v;
            v.x = acc[i][j][0] * f; v.y = acc[i][j][1] * f;
            v.z = acc[i][j][2] * f; v.w = acc[i][j][3] * f;
            *reinterpret_cast<float4*>(crow + j * 16 + lg * 4) = v;
          }
        }
      }
    } else {
      // stage the bf16 tile in LDS, then write whole rows with 16-byte stores
      constexpr int ld = kSilu ? kCtLdSilu : kCtLdStore;
      uint16_t* ct = reinterpret_cast<uint16_t*>(smem);
      __syncthreads();  // every wave is done reading the stages
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i < live_sub) {
          uint16_t* crow = ct + (wave_row0 + i * 16 + l16) * ld;
          if constexpr (kSilu) {
            const float fg = fac(i, 0), fu = fac(i, 1);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              float hv[4];
#pragma unroll
              for (int q = 0; q < 4; ++q) hv[q] = silu(acc[i][j][q] * fg) * (acc[i][j + 2][q] * fu);
              uint2 v;
              v.x = pack_bf16x2(hv[0], hv[1]);
              v.y = pack_bf16x2(hv[2], hv[3]);
              *reinterpret_cast<uint2*>(crow + wg * 32 + j * 16 + lg * 4) = v;
            }
          } else {
            const float f = fac(i, 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              uint2 v;
              v.x = pack_bf16x2(acc[i][j][0] * f, acc[i][j][1] * f);
              v.y = pack_bf16x2(acc[i][j][2] * f, acc[i][j][3] * f);
              *reinterpret_cast<uint2*>(crow + wg * 64 + j * 16 + lg * 4) = v;
            }
          }
        }
      }
      __syncthreads();
      if constexpr (EPI == Epi::kStoreBf16) {
        // 32 x 16-byte chunks per 256-column row
        const int c = tid & 31;
        for (int r = tid >> 5; r < valid; r += kThreads / 32) {
          const uint4 v = *reinterpret_cast<const uint4*>(ct + r * ld + c * 8);
          *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out +
                                    nt * kBN + c * 8) = v;
        }
      } else {
        // two threads per row, 64 columns each
        const int r = tid >> 1, half = tid & 1;
        const uint16_t* src = ct + r * ld + half * 64;
        float m = 0.0f;
        if (r < valid) {
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const uint4 v = *reinterpret_cast<const uint4*>(src + u * 8);
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q)
              m = fmaxf(m, fmaxf(fabsf(bf16_bits_to_f32(w[q] & 0xffffu)), fabsf(bf16_bits_to_f32(w[q] >> 16))));
          }
        }
        if constexpr (EPI == Epi::kSiluBf16) {
          if (r < valid) {
            uint16_t* dst = static_cast<uint16_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out + nt * 128 + half * 64;
#pragma unroll
            for (int u = 0; u < 8; ++u)
              *reinterpret_cast<uint4*>(dst + u * 8) = *reinterpret_cast<const uint4*>(src + u * 8);
          }
          m = wave_max(m);
          if (lane == 0 && p.amax != nullptr)
            atomicMax(reinterpret_cast<unsigned int*>(p.amax), __float_as_uint(m));
        } else if constexpr (EPI == Epi::kSiluMx) {
          // MX requantisation of the bf16 h: per row and 32-column block,
          // e = exponent field of amax (clamped to 254), q = e4m3(h * 2^(127-e))
          // (the quant_mx_kernel rule).  The tile's 128 columns are one K step
          // (nt) of the next GEMM; the block exponents of its rows are gathered
          // in LDS and written as that GEMM's packed words of M tile mnat
          // (word q, byte g: row 64*(q/64) + 16g + q%16, block (q%64)/16).
          uint8_t* ex = smem + kBM * kCtLdSilu * 2;  // [256 rows][4 blocks]
          uint8_t* dst = static_cast<uint8_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out + nt * 128 + half * 64;
#pragma unroll
          for (int b = 0; b < 2; ++b) {
            uint32_t ebits = 0;
            if (r < valid) {
              uint4 v[4];
              float am = 0.0f;
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                v[u] = *reinterpret_cast<const uint4*>(src + b * 32 + u * 8);
                const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
                for (int q = 0; q < 4; ++q)
                  am = fmaxf(am, fmaxf(fabsf(bf16_bits_to_f32(w[q] & 0xffffu)), fabsf(bf16_bits_to_f32(w[q] >> 16))));
              }
              ebits = min((__float_as_uint(am) >> 23) & 0xffu, 254u);
              const int sh = 127 - static_cast<int>(ebits);
              auto qv = [&](uint32_t h) { return __builtin_amdgcn_ldexpf(bf16_bits_to_f32(h), sh); };
              uint32_t qw[8];
#pragma unroll
              for (int u = 0; u < 4; ++u) {
                qw[2 * u] = pack_e4m3x4(qv(v[u].x & 0xffffu), qv(v[u].x >> 16), qv(v[u].y & 0xffffu), qv(v[u].y >> 16));
                qw[2 * u + 1] = pack_e4m3x4(qv(v[u].z & 0xffffu), qv(v[u].z >> 16), qv(v[u].w & 0xffffu), qv(v[u].w >> 16));
              }
              *reinterpret_cast<uint4*>(dst + b * 32) = uint4{qw[0], qw[1], qw[2], qw[3]};
              *reinterpret_cast<uint4*>(dst + b * 32 + 16) = uint4{qw[4], qw[5], qw[6], qw[7]};
            }
            ex[r * 4 + half * 2 + b] = static_cast<uint8_t>(ebits);  // 0 for rows past valid
          }
          __syncthreads();
          if (tid < kBM) {
            const int q = tid;
            const int rr = (q & ~63) + (q & 15), ks = (q >> 4) & 3;
            uint32_t w = 0;
#pragma unroll
            for (int g = 0; g < 4; ++g) w |= static_cast<uint32_t>(ex[(rr + 16 * g) * 4 + ks]) << (8 * g);
            reinterpret_cast<uint32_t*>(p.c_scale)[static_cast<int64_t>(nt) * p.cs_rs + static_cast<int64_t>(mnat) * kBM + q] = w;
          }
        } else {
          // 1x128 group = the row's 128 columns of this tile
          m = fmaxf(m, __shfl_xor(m, 1, 64));
          if (r < valid) {
            const float s = scale_from_amax(m);
            const float inv = 1.0f / s;
            uint8_t* dst = static_cast<uint8_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out + nt * 128 + half * 64;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              uint32_t qw[4];
#pragma unroll
              for (int h2 = 0; h2 < 2; ++h2) {
                const uint4 v = *reinterpret_cast<const uint4*>(src + u * 16 + h2 * 8);
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                  const uint32_t lo = w[2 * q], hi = w[2 * q + 1];
                  qw[h2 * 2 + q] = pack_e4m3x4(quot_e4m3(bf16_bits_to_f32(lo & 0xffffu), s, inv),
                                               quot_e4m3(bf16_bits_to_f32(lo >> 16), s, inv),
                                               quot_e4m3(bf16_bits_to_f32(hi & 0xffffu), s, inv),
                                               quot_e4m3(bf16_bits_to_f32(hi >> 16), s, inv));
                }
              }
              *reinterpret_cast<uint4*>(dst + u * 16) = uint4{qw[0], qw[1], qw[2], qw[3]};
            }
            if (half == 0) p.c_scale[static_cast<int64_t>(nt) * p.rows + row0 + r] = s;
          }
        }
      }
    }
  }
}

// Packed weight layout (a load-time transform; the grouped GEMMs then stream
// every weight panel sequentially instead of 128 bytes from each of 256 rows
// 7-14 KiB apart).  For expert e, 256-row N tile nt and K step kt the 32 KiB
// block at ((e*(nb/256) + nt)*(K/128) + kt)*32 KiB holds the tile's sixteen
// 16-row MFMA fragments in operand-register order ("fragment-major"):
//   block[f*2048 + h*1024 + l*16 + b] = w[e][wrow(16f + l%16)][kt*128 + (2*(l/16) + h)*16 + b],
// i.e. lane l's registers 0-3 (h = 0) and 4-7 (h = 1) of fragment f, so one
// 64-lane 16-byte load of 1 KiB contiguous bytes fills one register half of a
// fragment (the narrow kernel), and the 256x256 kernel copies the block
// linearly into LDS and reads each fragment half as 64 consecutive 16-byte
// chunks.  wrow(R) = nt*256 + R, or with gate_up = I (fused gate/up weights
// [gate I rows | up I rows]) the 64-row quarter R>>6 holds 32 gate rows then
// the 32 matching up rows:
//   wrow(R) = nt*128 + 32*(R>>6) + (R&31) + ((R>>5)&1)*I.
// One thread moves one 16-byte chunk; writes are linear.
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ w, int64_t nb,
                                                           int K, int gate_up, uint8_t* __restrict__ out,
                                                           int64_t chunks) {
  const int ks = K / kBK;
  const int64_t ntile = nb / kBN;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < chunks;
       c += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t blk = c >> 11;  // 2048 chunks per 32 KiB block
    const int in = static_cast<int>(c & 2047);
    const int f = in >> 7, h = (in >> 6) & 1, l = in & 63;
    const int R = 16 * f + (l & 15);
    const int chunk = 2 * (l >> 4) + h;
    const int kt = static_cast<int>(blk % ks);
    const int64_t tile = blk / ks;
    const int64_t e = tile / ntile;
    const int nt = static_cast<int>(tile - e * ntile);
    const int64_t wrow = gate_up ? nt * 128 + 32 * (R >> 6) + (R & 31) + ((R >> 5) & 1) * gate_up
                                 : static_cast<int64_t>(nt) * kBN + R;
    const uint8_t* src = w + (e * nb + wrow) * K + kt * kBK + (chunk << 4);
    *reinterpret_cast<uint4*>(out + (c << 4)) = *reinterpret_cast<const uint4*>(src);
  }
}

}  // namespace hkmoe
