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

#include <type_traits>

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
constexpr int kScaleBytes = kBM * 4;                     // activation scales (or MX words) of one K block
constexpr int kStageBytes = 2 * kTileBytes + kScaleBytes;
constexpr int kMaxKBlocks = 128;                         // K <= 16384
// LDS: two operand stages (in MX mode each 1 KiB larger, for the B exponent
// words), then
//   weight scales of two tiles (current / next)  [2][2 column blocks][kMaxKBlocks] fp32
//   gathered A rows of the next tile             [256] int32
//   epilogue scratch                             row maxima [256][4] fp32, or MX exponents
//   tile slots                                   [0, 1] first tile (m, n); [2..7] next tile
//                                                (m, n, expert, first row, rows, MX M tile)
// The epilogue stages its output tile in the A half of the last K step's
// stage (nothing else is live there) and this scratch, so the next tile's
// first stages can be in flight while it runs.
constexpr int kStageMax = kStageBytes + kScaleBytes;
// K-step variants of the persistent kernel: which next-tile work a step carries
constexpr int kPlain = 0, kClaim = 1, kLookup = 2, kPublish = 3, kStage = 4, kNextB0 = 5, kNextA0 = 6;
constexpr int kBsOff = 2 * kStageMax;
constexpr int kRowsOff = kBsOff + 2 * 2 * kMaxKBlocks * 4;
constexpr int kEpiOff = kRowsOff + kBM * 4;
constexpr int kSlotOff = kEpiOff + kBM * 4 * 4;
constexpr int kLdsBytes = kSlotOff + 32;

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

// Tile row of activation-scale slot s.  A group's 128 slots are two runs of
// 64: slots 4*l16 .. 4*l16 + 3 of the first run hold the scales of rows l16,
// 16 + l16, 32 + l16, 48 + l16 (sub-tiles 0-3 of the lane with that l16), the
// second run those of sub-tiles 4-7.  Each memory phase then reads one 16-byte
// chunk per l16 from 256 consecutive bytes: no two of the 16 addresses share a
// bank (the earlier 8-float runs put l16 and l16 + 8 in the same banks).
__device__ __forceinline__ int scale_slot_row(int slot) {
  const int wm = slot >> 7, w = slot & 127;
  return wm * 128 + ((w >> 6) * 4 + (w & 3)) * 16 + ((w & 63) >> 2);
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

// Wait for this wave's LDS reads (and its DMA: all of it, or all but the 4
// newest loads), then the workgroup barrier; memory operations stay on their
// side of it.  TRACKED: the compiler's own s_waitcnt (simm16: vmcnt in bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8) between empty asm statements with
// a memory clobber, so its wait tracking knows which loads the wait covered
// and adds no vmcnt(0) of its own where the register of an older load (the
// next tile's claim and lookups) is used later; otherwise one asm statement,
// which it cannot see into.  Tracked, the gate/up GEMM with block scales is
// 1.0-1.4% faster and the per-tensor one 0.5%; the bf16-store and MX GEMMs
// measured slower tracked (+0.8-1.5%, +0.8%) and keep the asm form.
constexpr int kWaitVm0Lgkm0 = 0x0070;  // s_waitcnt vmcnt(0) lgkmcnt(0)
constexpr int kWaitVm4Lgkm0 = 0x0074;  // s_waitcnt vmcnt(4) lgkmcnt(0)
constexpr int kWaitLgkm0 = 0xC07F;     // s_waitcnt lgkmcnt(0)
template <bool TRACKED, int WAIT>
__device__ __forceinline__ void wait_barrier() {
  static_assert(WAIT == kWaitVm0Lgkm0 || WAIT == kWaitVm4Lgkm0 || WAIT == kWaitLgkm0, "wait");
  if constexpr (TRACKED) {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  } else if constexpr (WAIT == kWaitVm4Lgkm0) {
    asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else if constexpr (WAIT == kWaitVm0Lgkm0) {
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  } else {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
}

// B source of the tile (expert e, N tile nt) for one wave: buffer descriptor,
// lane offset within a K step, and the K-step stride (see the B layout notes
// in gemm_fp8_persistent).  A plain function with scalar parameters: in a
// lambda the same code made the compiler keep lane constants in private memory.
__device__ __forceinline__ void b_source(const GemmParams& p, int e, int nt, bool silu, int wg, i32x4& srd,
                                         int& voff, int& kstride) {
  const int lane = lane_here();
  if (p.b_packed) {
    // K step kt of N tile nt: block (e, kt, nt), nb/256 blocks per K step
    srd = make_srd(p.b + static_cast<int64_t>(e) * p.nb * p.K + static_cast<int64_t>(nt) * kTileBytes,
                   static_cast<uint32_t>(static_cast<int64_t>(p.nb) * p.K - static_cast<int64_t>(nt) * kTileBytes));
    voff = wg * 8 * kBK + lane * 16;
    kstride = (p.nb / kBN) * kTileBytes;
  } else {
    srd = make_srd(p.b + static_cast<int64_t>(e) * p.nb * p.K, static_cast<uint32_t>(p.nb) * p.K);
    const int ld_row = 8 * wg + (lane >> 3), ld_chunk = (lane & 7) ^ swz(ld_row);
    const int b_row0 = silu ? nt * 128 + ld_row : nt * kBN + ld_row;
    voff = buf_off(b_row0, p.K, ld_chunk * 16);
    kstride = kBK;
  }
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wunused-lambda-capture"
template <Epi EPI, Scale SC>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_persistent(GemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  constexpr bool kBlockSc = (SC == Scale::kBlock);
  constexpr bool kMX = (SC == Scale::kMX);
  constexpr bool kSilu = (EPI == Epi::kSiluBf16 || EPI == Epi::kSiluQuant || EPI == Epi::kSiluMx);
  // barrier waits the compiler tracks (see wait_barrier): the gate/up GEMMs
  // with block and per-tensor scales
  constexpr bool kTrackedWaits = (EPI == Epi::kSiluQuant || EPI == Epi::kSiluBf16) && !kMX;
  auto sync_lds = []() __attribute__((always_inline)) { wait_barrier<kTrackedWaits, kWaitLgkm0>(); };
  // stage: A tile, B tile, A scales (1 KiB) and, in MX mode, B scales (1 KiB)
  constexpr int kStg = kMX ? kStageBytes + kScaleBytes : kStageBytes;
  // A sub-tiles of the first compute phase that it reads itself instead of
  // the first memory phase (block and per-tensor scales): that phase is bound
  // by its LDS reads (17 ds_read_b128 per wave against 9 in the second), while
  // in the compute phase the reads overlap the MFMAs and the other wave's
  // memory phase.  Sub-tiles 2 and 3 are read after MFMAs 1 and 5, in time for
  // their first use at MFMAs 8 and 12 (config-3 layer -0.3%, three sub-tiles
  // the same; Mixtral layer -0.7%; dense GEMMs unchanged).
  constexpr int kLateA = (kBlockSc || SC == Scale::kTensor) ? 2 : 0;
  static_assert(EPI != Epi::kSiluMx || kMX, "MX requantisation needs MX scales");
  static_assert(2 * kStg <= kBsOff, "LDS budget");

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
#define HK_SLOT reinterpret_cast<int*>(smem + kSlotOff)
#define HK_NROW reinterpret_cast<int*>(smem + kRowsOff)
#define HK_BS reinterpret_cast<float*>(smem + kBsOff)
  const int xcd = blockIdx.x & 7;
#define HK_CAP tid, wave, lane, grp, wg, l16, lg, wave_row0, fx, dense, total_mtiles, k_steps, ld_row, ld_chunk, xcd
  int steal = 0;       // thread 0: tile queues visited so far
  int static_j = vid;  // thread 0: the static schedule's next slot

  // ---- tile source (thread 0) ------------------------------------------------
  // With tile counters, slot j of queue q is tile (m, n) of block b = q + 8*(j/32);
  // a drained queue moves on to the next XCD's.  Without, the same blocks are
  // walked statically: the vid-th slot of every round of g slots.  A claim is
  // split in two: claim_start issues the atomic on the current queue and
  // claim_end, which may run a K step later, turns its slot into a tile (or
  // takes further slots: past a queue's end, or outside the tile grid).
  auto tile_of = [&, HK_CAP](int b, int sl, int& n) __attribute__((always_inline)) -> int {
    const int m = bm * (b / nbn) + (sl & (bm - 1));
    n = bn * (b % nbn) + (sl >> p.blk_m_log2);
    return (m < total_mtiles && n < p.n_tiles) ? m : -1;
  };
  auto queue_slots = [&, HK_CAP](int q) __attribute__((always_inline)) -> int {
    return q < nblocks ? 32 * ((nblocks - q + 7) >> 3) : 0;
  };
  auto claim_start = [&, HK_CAP]() __attribute__((always_inline)) -> int {
    if (p.tile_ctr == nullptr || steal >= 8) return 0;
    const int q = (xcd + steal) & 7;
    return queue_slots(q) > 0 ? atomicAdd(&p.tile_ctr[q], 1) : 0;
  };
  auto claim_end = [&, HK_CAP](int j, int& n) __attribute__((always_inline)) -> int {  // m, or -1
    if (p.tile_ctr == nullptr) {
      while (true) {
        const int js = static_j;
        static_j += g;
        if ((js >> 5) >= nblocks) return -1;
        const int m = tile_of(js >> 5, js & 31, n);
        if (m >= 0) return m;
      }
    }
    while (steal < 8) {
      const int q = (xcd + steal) & 7;
      if (j < queue_slots(q)) {
        const int m = tile_of(q + 8 * (j >> 5), j & 31, n);
        if (m >= 0) return m;
      } else {
        ++steal;
      }
      if (steal < 8) {
        const int q2 = (xcd + steal) & 7;
        j = queue_slots(q2) > 0 ? atomicAdd(&p.tile_ctr[q2], 1) : 0;
      }
    }
    return -1;
  };

  // ---- tile -> expert segment (uniform) ---------------------------------------
  struct Tile {
    int t, nt, e, row0, valid, mnat;  // t: M tile (-1: none); mnat: M tile in expert order
  };
  // (expert, first row, rows, MX M tile) of M tile m, from the routing tables
  auto locate = [&, HK_CAP](int m, int& e, int& row0, int& valid, int& mnat) __attribute__((always_inline)) {
    e = 0;
    mnat = m;
    if (dense) {
      row0 = m * kBM;
      valid = static_cast<int>(min<int64_t>(kBM, p.rows - row0));
    } else if (p.mtile_list != nullptr) {
      e = p.mtile_list[2 * m];
      row0 = p.mtile_list[2 * m + 1];
      valid = min(kBM, p.offsets[e + 1] - row0);
      if constexpr (kMX) mnat = p.mtile_offsets[e] + (row0 - p.offsets[e]) / kBM;
    } else {
      int lo = 0, hi = p.num_experts;  // largest e with mtile_offsets[e] <= m
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (p.mtile_offsets[mid] <= m) lo = mid; else hi = mid;
      }
      e = lo;
      row0 = p.offsets[e] + (m - p.mtile_offsets[e]) * kBM;
      valid = min(kBM, p.offsets[e + 1] - row0);
    }
  };
  auto uniform = [](int m, int n, int e, int row0, int valid, int mnat) __attribute__((always_inline)) {
    Tile c{-1, 0, 0, 0, 0, 0};
    c.t = __builtin_amdgcn_readfirstlane(m);
    if (c.t < 0) return c;
    c.nt = __builtin_amdgcn_readfirstlane(n);
    c.e = __builtin_amdgcn_readfirstlane(e);
    c.row0 = __builtin_amdgcn_readfirstlane(row0);
    c.valid = __builtin_amdgcn_readfirstlane(valid);
    c.mnat = __builtin_amdgcn_readfirstlane(mnat);
    return c;
  };
  // the tile (m, n) published in LDS slots s, s + 1, located here
  auto decode = [&, HK_CAP](int s) __attribute__((always_inline)) {
    const int m = __builtin_amdgcn_readfirstlane(HK_SLOT[s]);
    if (m < 0) return Tile{-1, 0, 0, 0, 0, 0};
    int e, row0, valid, mnat;
    locate(m, e, row0, valid, mnat);
    return uniform(m, HK_SLOT[s + 1], e, row0, valid, mnat);
  };

  // Lane offsets of the two register halves of a B fragment within its 2 KiB
  // of the stage: fragment-major (packed weights) or swizzled rows, in the K
  // order of the MFMA variant (read_frag / read_frag_mx).
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

  // ---- per-tile DMA sources --------------------------------------------------
  // B (group 0 rows 0-127, group 1 rows 128-255): LDS row 32*i + ld_row holds
  // weight row b_row0 + boff(i)
  //   plain: nt*256 + r                       -> boff(i) = 32*i
  //   SiLU:  quarter q = r >> 6 = i >> 1 holds 32 gate rows (i even) then
  //          the 32 matching up rows (i odd) -> boff(i) = 32*(i>>1) + (i&1)*I
  // Row-major weights: lane offset of that row and chunk, K step kt at byte
  // kt*128.  Packed weights: the tile's K step kt is the 32 KiB stage image at
  // kt*32 KiB of the tile's own panel, so instruction i of wave wg reads the
  // 1 KiB at (32*i + 8*wg)*128 linearly.
  i32x4 b_srd;
  int b_voff = 0, b_kstride = 0;
#define HK_SET_B(c) b_source(p, (c).e, (c).nt, kSilu, wg, b_srd, b_voff, b_kstride)
  // A (own half): LDS row grp*128 + 32*i + ld_row <- A row of output row
  // row0 + min(r, valid - 1); 16-row sub-tiles past `valid` are not loaded.
  // Gathered rows come straight from a_gather, or, for a tile prepared during
  // the previous tile's K loop, from its row list in LDS (stage_rows).
  // The activation-scale loaders (waves 0, 1 of each group, block scales)
  // gather 64 slots of the own half; MX: wave 0 DMAs the tile's 256 A words of
  // a K step (1 KiB), wave 1 its 256 B words, words past the packed arrays
  // read as zero (rows that are never stored).
  const bool scale_loader = kBlockSc && wg < 2;
  const bool mx_loader = kMX && wave < 2;
  int a_voff[4], as_voff = 0, mx_voff = 0, mx_kstride = 0, mx_lds = 0;
  i32x4 mx_srd = {0, 0, 0, 0};
  auto a_row = [&, HK_CAP](const Tile& c, int r, bool staged) __attribute__((always_inline)) -> int {
    const int rc = min(r, c.valid - 1);
    if (p.a_gather == nullptr) return c.row0 + rc;
    return (staged ? HK_NROW[rc] : p.a_gather[c.row0 + rc]) / p.gather_div;
  };
  auto set_a = [&, HK_CAP](const Tile& c, bool staged) __attribute__((always_inline)) {
    // lane constants recomputed here (once per tile)
    const int ln = lane_here();
    const int lrow = 8 * wg + (ln >> 3), lchunk = (ln & 7) ^ swz(lrow);
#pragma unroll
    for (int i = 0; i < 4; ++i) a_voff[i] = buf_off(a_row(c, wave_row0 + 32 * i + lrow, staged), p.K, lchunk * 16);
    if (scale_loader)
      as_voff = static_cast<int>(a_row(c, scale_slot_row(wave_row0 + wg * 64 + ln), staged) * p.as_rs) * 4;
    if constexpr (kMX) {
      if (wave == 0) {
        mx_srd = make_srd(p.a_scale, static_cast<uint32_t>(k_steps * p.as_rs * 4));
        mx_voff = (c.mnat * kBM + ln * 4) * 4;
        mx_kstride = static_cast<int>(p.as_rs) * 4;
        mx_lds = 2 * kTileBytes;
      } else if (wave == 1) {
        if (dense) {
          mx_srd = make_srd(p.b_scale, static_cast<uint32_t>(k_steps * p.nb * 4));
          mx_voff = (c.nt * kBN + ln * 4) * 4;
          mx_kstride = p.nb * 4;
        } else {
          // this B tile's words: k_steps consecutive KiB
          const int ntiles = p.nb / kBN;
          mx_srd = make_srd(reinterpret_cast<const uint8_t*>(p.b_scale) +
                                (static_cast<int64_t>(c.e) * ntiles + c.nt) * k_steps * 1024,
                            static_cast<uint32_t>(k_steps) * 1024);
          mx_voff = ln * 16;
          mx_kstride = 1024;
        }
        mx_lds = 2 * kTileBytes + kScaleBytes;
      }
    }
  };
  // The next tile's gathered rows into LDS: waves 0-3, 64 row indices each.
  auto stage_rows = [&, HK_CAP](const Tile& c) __attribute__((always_inline)) {
    if (p.a_gather != nullptr && wave < 4) {
      const i32x4 g_srd = make_srd(p.a_gather, 0xffffffffu);
      load_lds_4B(g_srd, HK_NROW + 64 * wave, (c.row0 + min(64 * wave + lane_here(), c.valid - 1)) * 4, 0);
    }
  };
  // A tile's weight scales for every K step into buffer `buf`: waves 0-3, one
  // column block (gate / first, up / second) and 64 K steps each; steps past
  // K read as zero.
  auto stage_bscales = [&, HK_CAP](const Tile& c, int buf) __attribute__((always_inline)) {
    if constexpr (kBlockSc) {
      const int h = wave & 1, part = wave >> 1;
      if (wave < 4 && part * 64 < k_steps) {
        const int nbh = h ? (kSilu ? p.n_out / kGroup + c.nt : 2 * c.nt + 1) : (kSilu ? c.nt : 2 * c.nt);
        const float* src = p.b_scale + (static_cast<int64_t>(c.e) * (p.nb / kGroup) + nbh) * k_steps;
        const i32x4 srd = make_srd(src, static_cast<uint32_t>(k_steps) * 4);
        load_lds_4B(srd, HK_BS + (buf * 2 + h) * kMaxKBlocks + part * 64, (part * 64 + lane_here()) * 4, 0);
      }
    }
  };

  // DMA instructions of one K step issued by this wave.  issue_a: its group's
  // A half of K step kt of a tile of `valid` rows into stage stg (4, dead
  // 16-row sub-tiles skipped) and, for the scale / MX loaders, one more.
  // issue_b: exactly 4 loads, half of the B stage (group 0 rows 0-127, group 1
  // rows 128-255); being the last 4 loads a wave issues in a K step, they are
  // what vmcnt(4) leaves in flight.
  auto issue_a = [&, HK_CAP](int kt, int stg, int valid) __attribute__((always_inline)) {
    uint8_t* sa = smem + stg * kStg;
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
  auto issue_b = [&, HK_CAP](int kt, int stg) __attribute__((always_inline)) {
    uint8_t* sb = smem + stg * kStg + kTileBytes;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int i = grp * 4 + q;
      const int boff = kSilu ? (32 * (i >> 1) + ((i & 1) ? p.n_out : 0)) : 32 * i;
      const int ioff = p.b_packed ? 32 * i * kBK : buf_off(boff, p.K, 0);
      load_lds_16B(b_srd, sb + (32 * i + 8 * wg) * kBK, b_voff, kt * b_kstride + ioff);
    }
  };
  // every load of this wave except its last issue_b has completed
  auto wait_dma = [&, HK_CAP](bool b_in_flight) __attribute__((always_inline)) {
    if (b_in_flight) wait_barrier<kTrackedWaits, kWaitVm4Lgkm0>();
    else wait_barrier<kTrackedWaits, kWaitVm0Lgkm0>();
  };
  // a tile's first two stages (steps 0 and 1 at global steps gs, gs + 1) and
  // its weight scales, when the previous tile did not prepare them
  auto start_tile = [&, HK_CAP](const Tile& c, int buf, int gs) __attribute__((always_inline)) {
    HK_SET_B(c);
    set_a(c, false);
    stage_bscales(c, buf);
    issue_a(0, gs & 1, c.valid);
    issue_b(0, gs & 1);
    if (k_steps > 1) issue_b(1, (gs + 1) & 1);
    wait_dma(k_steps > 1);  // stage 0 and the weight scales visible to all
  };

  // The next tile is found during a tile's K loop by thread 0, one memory
  // round trip per K step, each looked at only after the step's own DMA wait
  // (which covers it): the slot's atomic was issued before the tile began;
  // step 1's end turns the slot into (m, n) and loads the M tile's (expert,
  // first row); step 2's end loads the
  // expert's row offsets; step 3's end publishes the tile in LDS.  Step
  // k_steps - 3 reads it and DMAs its gathered rows and weight scales into
  // LDS; its first stages are loaded by the last K steps like any other step:
  // B(0) at step k_steps - 2, A(0) and B(1) at k_steps - 1.  Stage parity runs
  // on a global step count, so it continues across tiles.  With fewer than 8
  // K steps each tile starts on its own after the previous epilogue.
  const bool pipe = k_steps >= 8;
  if (tid == 0) {
    int n = 0;
    HK_SLOT[0] = claim_end(claim_start(), n);
    HK_SLOT[1] = n;
  }
  __syncthreads();
  Tile cur = decode(0);
  if (cur.t < 0) return;
  int buf = 0, gstep = 0;
  start_tile(cur, buf, gstep);
  // thread 0: the claim slot that step 1 of the current tile turns into the
  // next tile.  With kEarlyClaim its atomic is issued before the tile starts
  // (here, then at the end of each epilogue), so it has two K steps to return
  // instead of one; it pays where tiles are short (GEMM 2: 16 K steps, 2.7%),
  // while in GEMM 1 the register it keeps across the tile loop cost more
  // (+1.8%: scalar spills reached the loop of plain steps), so there step 1
  // issues it.
  constexpr bool kEarlyClaim = (EPI == Epi::kStoreBf16);
  int q_j_next = 0;
  if (kEarlyClaim && pipe && tid == 0) q_j_next = claim_start();

  while (true) {
    if (grp == 1) sync_lds();  // group 1 runs one phase behind group 0
    const float* bsl = HK_BS + buf * 2 * kMaxKBlocks;
    const int live_sub = max(0, min(8, (cur.valid - wave_row0 + 15) >> 4));
    Tile nxt{-1, 0, 0, 0, 0, 0};
    // thread 0's lookups of the next tile (meaningful in lane 0 only)
    int q_j = q_j_next, q_m = -1, q_n = 0, q_e = 0, q_row0 = 0, q_end = 0, q_beg = 0, q_mt = 0;

    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // block scales of the current K step: the activation scales of the lane's 4
    // sub-tile rows of the coming compute phase, and the weight scale of its
    // gate / up (or only) 128-column block
    float sa_cur[4], sb_cur0 = 1.0f, sb_cur1 = 1.0f;

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
    // One K step.  kPlain: this tile's loads only (A(kt+1), B(kt+2) while
    // they exist); with pipelining, kClaim / kLookup / kPublish: steps 1-3,
    // which find the next tile (thread 0); kStage: step k_steps-3, which reads
    // it and stages its rows and weight scales; kNextB0: step k_steps-2, whose
    // B load is the next tile's B(0) and which sets up the next tile's A
    // sources; kNextA0: the last step, whose loads are the next tile's A(0) and
    // B(1).  The steps with next-tile work are separate copies, so the loop of
    // plain steps keeps the registers of a single tile.
    auto step = [&, HK_CAP](int kt, auto mode_tag) __attribute__((always_inline)) {
      constexpr int MODE = decltype(mode_tag)::value;
      const int stg = (gstep + kt) & 1;
      const uint8_t* sa = smem + stg * kStg;
      const uint8_t* sb = sa + kTileBytes;
      if constexpr (MODE == kNextA0) {
        // first thing: the next tile's A(0) (its sources were set a step ago)
        // into the previous step's stage, whose reads all ended with that step
        if (nxt.t >= 0) issue_a(0, stg ^ 1, nxt.valid);
      }
      if constexpr (MODE == kClaim && !kEarlyClaim) {
        if (tid == 0) q_j = claim_start();
      }
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
        for (int i = 0; i < 4 - kLateA; ++i) af[i] = read_operand<kMX>(sa, wave_row0 + i * 16 + l16, lg, fx);
      }
      if constexpr (kBlockSc) {
        // this step's scales of sub-tiles 0-3 (4-7 in the second memory phase);
        // the factors are formed in the compute phases
        const f32x4 s_lo = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(sb + kTileBytes) +
                                                           wave_row0 + l16 * 4);
        sa_cur[0] = s_lo.x; sa_cur[1] = s_lo.y; sa_cur[2] = s_lo.z; sa_cur[3] = s_lo.w;
        if constexpr (kSilu) {
          sb_cur0 = bsl[kt];
          sb_cur1 = bsl[kMaxKBlocks + kt];
        } else {
          sb_cur0 = sb_cur1 = bsl[(wg >> 1) * kMaxKBlocks + kt];
        }
      }
      if constexpr (MODE != kNextA0) {
        if (MODE != kPlain || kt + 1 < k_steps) issue_a(kt + 1, stg ^ 1, cur.valid);
      }
      if constexpr (MODE == kStage) {
        // the next tile, published at step 3: its rows and weight scales into LDS
        nxt = uniform(HK_SLOT[2], HK_SLOT[3], HK_SLOT[4], HK_SLOT[5], HK_SLOT[6], HK_SLOT[7]);
        if (nxt.t >= 0) {
          stage_rows(nxt);
          stage_bscales(nxt, buf ^ 1);
        }
      }
      if constexpr (MODE == kNextB0) {
        // this tile's last A load is issued: the A sources become the next tile's
        // (its rows were staged a step ago)
        if (nxt.t >= 0) set_a(nxt, true);
      }
      sync_lds();
      __builtin_amdgcn_sched_barrier(0);

      // ---- compute phase 1: sub-tiles 0-3
      auto compute = [&, HK_CAP](int i0) __attribute__((always_inline)) {
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
            // MFMA t from zero; the FMAs folding MFMA t-2 into its accumulator
            // follow it, so they run while MFMA t occupies the matrix core and
            // read a result two MFMAs old (folding the previous MFMA's result
            // stalls on it: about 44 instead of 38 cycles per MFMA).  The order
            // is pinned with scheduling groups.  Factor of sub-tile u: its row's
            // activation scale times the weight scale of the column block
            // (gate: j < 2, up: j >= 2), formed before its first fold.
            f32x4 pr[3];
            float f0 = 0.0f, f1 = 0.0f;
#pragma unroll
            for (int t = 0; t < 18; ++t) {
              if (t < 16) pr[t % 3] = mfma_e4m3_16x16x128(bf[t & 3], af[t >> 2], f32x4{0.f, 0.f, 0.f, 0.f});
              // the first compute phase reads its last kLateA A sub-tiles here,
              // a few MFMAs before their first use (sub-tile u at MFMA 4u)
              if (i0 == 0 && kLateA > 0 && (t == 1 || t == 5) && (t == 5 || kLateA == 2)) {
                const int u = (t == 1) ? 2 : 3;
                af[u] = read_operand<kMX>(sa, wave_row0 + u * 16 + l16, lg, fx);
              }
              if (t >= 2) {
                const int u = (t - 2) >> 2, j = (t - 2) & 3;
                if (j == 0) {
                  f0 = sa_cur[u] * sb_cur0;
                  f1 = kSilu ? sa_cur[u] * sb_cur1 : f0;
                }
                fold_block(acc[i0 + u][j], pr[(t - 2) % 3], (kSilu && j >= 2) ? f1 : f0);
              }
              if (t < 16) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA, then the VALU
              if (t >= 2 && ((t - 2) & 3) == 0) __builtin_amdgcn_sched_group_barrier(0x002, kSilu ? 6 : 5, 0);
              if (t >= 2 && ((t - 2) & 3) != 0) __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
              if (i0 == 0 && kLateA > 0 && (t == 1 || t == 5) && (t == 5 || kLateA == 2))
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // its two LDS reads
            }
          } else {
#pragma unroll
            for (int t = 0; t < 16; ++t) {
              const int u = t >> 2, j = t & 3;
              acc[i0 + u][j] = mfma_e4m3_16x16x128(bf[j], af[u], acc[i0 + u][j]);
              if (i0 == 0 && kLateA > 0 && (t == 1 || t == 5) && (t == 5 || kLateA == 2)) {
                const int ul = (t == 1) ? 2 : 3;
                af[ul] = read_operand<kMX>(sa, wave_row0 + ul * 16 + l16, lg, fx);
              }
              if (kLateA > 0 && i0 == 0) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if ((t == 1 || t == 5) && (t == 5 || kLateA == 2)) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
              }
            }
          }
        }
        __builtin_amdgcn_s_setprio(0);
      };
      compute(0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);

      // ---- memory phase 2: A sub-tiles 4-7 and their scales, B two steps
      // ahead (the next tile's B(0) / B(1) at the last two steps)
      if constexpr (kBlockSc) {
        const f32x4 s_hi = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(sb + kTileBytes) +
                                                           wave_row0 + 64 + l16 * 4);
        sa_cur[0] = s_hi.x; sa_cur[1] = s_hi.y; sa_cur[2] = s_hi.z; sa_cur[3] = s_hi.w;
      }
      if (live_sub > 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) af[i] = read_operand<kMX>(sa, wave_row0 + (i + 4) * 16 + l16, lg, fx);
      }
      bool b_fly = false;
      if constexpr (MODE == kNextB0 || MODE == kNextA0) {
        if (nxt.t >= 0) {
          if constexpr (MODE == kNextB0) HK_SET_B(nxt);  // this tile's B loads are done
          issue_b(MODE == kNextB0 ? 0 : 1, stg);
          b_fly = true;
        }
      } else if (MODE != kPlain || kt + 2 < k_steps) {
        issue_b(kt + 2, stg);
        b_fly = true;
      }
      if (grp == 1) wait_dma(b_fly); else sync_lds();
      __builtin_amdgcn_sched_barrier(0);

      // ---- compute phase 2: sub-tiles 4-7
      compute(4);
      __builtin_amdgcn_sched_barrier(0);
      if (grp == 0) wait_dma(b_fly); else __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);

      // thread 0's lookups: each result was covered by this step's DMA wait
      if constexpr (MODE == kClaim) {
        if (tid == 0) {
          q_m = claim_end(q_j, q_n);
          if (q_m >= 0 && !dense && p.mtile_list != nullptr) {
            q_e = p.mtile_list[2 * q_m];
            q_row0 = p.mtile_list[2 * q_m + 1];
          }
        }
      } else if constexpr (MODE == kLookup) {
        if (tid == 0 && q_m >= 0 && !dense && p.mtile_list != nullptr) {
          q_end = p.offsets[q_e + 1];
          if constexpr (kMX) {
            q_beg = p.offsets[q_e];
            q_mt = p.mtile_offsets[q_e];
          }
        }
      } else if constexpr (MODE == kPublish) {
        // read at step k_steps - 3 >= 5, after this step's barriers
        if (tid == 0) {
          int e = q_e, row0 = q_row0, valid = 0, mnat = q_m;
          if (q_m >= 0) {
            if (!dense && p.mtile_list != nullptr) {
              valid = min(kBM, q_end - row0);
              if constexpr (kMX) mnat = q_mt + (row0 - q_beg) / kBM;
            } else {
              locate(q_m, e, row0, valid, mnat);
            }
          }
          HK_SLOT[2] = q_m; HK_SLOT[3] = q_n; HK_SLOT[4] = e;
          HK_SLOT[5] = row0; HK_SLOT[6] = valid; HK_SLOT[7] = mnat;
        }
      }
    };
    if (pipe) {
      step(0, std::integral_constant<int, kPlain>{});
      step(1, std::integral_constant<int, kClaim>{});
      step(2, std::integral_constant<int, kLookup>{});
      step(3, std::integral_constant<int, kPublish>{});
      for (int kt = 4; kt < k_steps - 3; ++kt) step(kt, std::integral_constant<int, kPlain>{});
      step(k_steps - 3, std::integral_constant<int, kStage>{});
      step(k_steps - 2, std::integral_constant<int, kNextB0>{});
      step(k_steps - 1, std::integral_constant<int, kNextA0>{});
    } else {
      for (int kt = 0; kt < k_steps; ++kt) step(kt, std::integral_constant<int, kPlain>{});
    }
    if (grp == 0) sync_lds();  // group 0's extra barrier pairs with group 1's first
    // without pipelining the next tile is claimed now and started after the epilogue
    if (!pipe) {
      if (tid == 0) {
        int n = 0;
        HK_SLOT[0] = claim_end(claim_start(), n);
        HK_SLOT[1] = n;
      }
      __syncthreads();
      nxt = decode(0);
    }

    // ---- epilogue ------------------------------------------------------------
    // lane holds, for sub-tile i and n fragment j, output row wave_row0+16i+l16
    // and columns 16*j + 4*lg .. +3 of the wave's 64-column quarter; for the
    // SiLU epilogues fragments j and j+2 are the gate and up columns of h
    // columns 32*wg + 16*j + 4*lg .. +3 of the tile's 128.
    // `ct`: the A half of the last K step's stage (32 KiB), free until the next
    // tile's step 0 DMAs A(1) into it; output tiles are staged there and stored
    // as 16-byte chunks that cover whole rows.  Rows of 16-byte chunks; chunk c
    // of row r sits at slot c ^ (r mod the row's chunk count), so both the
    // fragment-shaped writes and the row-shaped reads spread over the banks.
    uint8_t* ct = smem + ((gstep + k_steps - 1) & 1) * kStg;
    const int row0 = cur.row0, valid = cur.valid, nt = cur.nt;
    // output rows row0 .. row0 + valid - 1 as one buffer: stores to rows past
    // `valid` (the next expert's rows) fall outside it and are dropped
    constexpr int kOutBytes = (EPI == Epi::kStoreBf16) ? 2 : (EPI == Epi::kSiluQuant || EPI == Epi::kSiluMx) ? 1 : 4;
    const i32x4 out_srd =
        make_srd(static_cast<uint8_t*>(p.c) + static_cast<int64_t>(row0) * p.n_out * kOutBytes,
                 static_cast<uint32_t>(valid) * static_cast<uint32_t>(p.n_out) * kOutBytes);
    // lane position recomputed here, so its address terms are not kept live
    // from the kernel's start
    const int eln = lane_here(), el16 = eln & 15, elg = eln >> 4;
    // per-tensor scales are applied here; block-scaled and MX accumulators
    // already hold the scaled sums
    float tens = 1.0f;
    if constexpr (SC == Scale::kTensor)
      tens = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[cur.e] : 1.0f);

    if constexpr (EPI == Epi::kStoreBf16) {
      // four rounds of 64 rows: sub-tiles 2q, 2q+1 of both halves (LDS row
      // rr = 32*grp + 16*(i - 2q) + l16, 512 bytes = 32 chunks)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (32 * q >= valid) break;  // uniform: no row of this round or later is stored
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = 2 * q + h, rr = grp * 32 + h * 16 + el16;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int c = wg * 8 + 2 * j + (elg >> 1);
            uint2 v;
            v.x = pack_bf16x2(acc[i][j][0] * tens, acc[i][j][1] * tens);
            v.y = pack_bf16x2(acc[i][j][2] * tens, acc[i][j][3] * tens);
            *reinterpret_cast<uint2*>(ct + rr * 512 + ((c ^ (rr & 31)) << 4) + (elg & 1) * 8) = v;
          }
        }
        sync_lds();
        // the four LDS reads, then four unconditional stores through a
        // descriptor that ends at the tile's last valid row (the hardware drops
        // the rows past it): the reads' latencies overlap, and no branch
        // separates them from the stores.  The output is not read again by
        // this kernel: non-temporal stores leave the L2 to the operand panels.
        uint4 sv[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int idx = wave * 64 + eln + kThreads * u, rr = idx >> 5, c = idx & 31;
          sv[u] = *reinterpret_cast<const uint4*>(ct + rr * 512 + ((c ^ (rr & 31)) << 4));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int idx = wave * 64 + eln + kThreads * u, rr = idx >> 5, c = idx & 31;
          const int r = (rr >> 5) * 128 + 32 * q + (rr & 31);
          store_16B<kAuxNT>(out_srd, (r * p.n_out + nt * kBN + c * 8) * 2, sv[u]);
        }
        sync_lds();
      }
    } else if constexpr (EPI == Epi::kStoreF32) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave_row0 + i * 16 + l16;
        if (i < live_sub && r < valid) {
          const int64_t off = static_cast<int64_t>(row0 + r) * p.n_out + nt * kBN + wg * 64 + lg * 4;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float4 v;
            v.x = acc[i][j][0] * tens; v.y = acc[i][j][1] * tens;
            v.z = acc[i][j][2] * tens; v.w = acc[i][j][3] * tens;
            *reinterpret_cast<float4*>(static_cast<float*>(p.c) + off + j * 16) = v;
          }
        }
      }
    } else {
      // h = bf16(SiLU(gate) * up): lane's 8 values of sub-tile i (h columns
      // 32*wg + 16*j + 4*lg .. +3 of row wave_row0 + 16i + l16, j = 0, 1)
      auto h_of = [&, HK_CAP](int i, int j) __attribute__((always_inline)) -> uint2 {
        float hv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) hv[q] = silu(acc[i][j][q] * tens) * (acc[i][j + 2][q] * tens);
        return uint2{pack_bf16x2(hv[0], hv[1]), pack_bf16x2(hv[2], hv[3])};
      };
      auto absmax = [](uint2 v) __attribute__((always_inline)) -> float {
        return fmaxf(fmaxf(fabsf(bf16_bits_to_f32(v.x & 0xffffu)), fabsf(bf16_bits_to_f32(v.x >> 16))),
                     fmaxf(fabsf(bf16_bits_to_f32(v.y & 0xffffu)), fabsf(bf16_bits_to_f32(v.y >> 16))));
      };
      // max |h| of the row over the wave's 32 columns (the 4 lane groups lg)
      auto wave_row_max = [](float m) __attribute__((always_inline)) -> float {
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        return fmaxf(m, __shfl_xor(m, 32, 64));
      };
      auto hcol = [&, HK_CAP](int j) __attribute__((always_inline)) { return nt * 128 + wg * 32 + j * 16 + lg * 4; };
      if constexpr (EPI == Epi::kSiluBf16) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = wave_row0 + i * 16 + l16;
          if (i < live_sub && r < valid) {
            uint16_t* dst = static_cast<uint16_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const uint2 v = h_of(i, j);
              *reinterpret_cast<uint2*>(dst + hcol(j)) = v;
              m = fmaxf(m, absmax(v));
            }
          }
        }
        m = wave_max(m);
        if (lane == 0 && p.amax != nullptr)
          atomicMax(reinterpret_cast<unsigned int*>(p.amax), __float_as_uint(m));
      } else if constexpr (EPI == Epi::kSiluMx) {
        // MX requantisation of h: per row and 32-column block (the wave's 32
        // columns), e = exponent field of amax (clamped to 254), q =
        // e4m3(h * 2^(127-e)) (the quant_mx_kernel rule).  The tile's 128
        // columns are one K step (nt) of the next GEMM; the block exponents of
        // its rows are collected in LDS and written as that GEMM's packed words
        // of M tile mnat (word q, byte g: row 64*(q/64) + 16g + q%16, block
        // (q%64)/16).
        uint8_t* ex = smem + kEpiOff;  // [256 rows][4 blocks]
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = wave_row0 + i * 16 + l16;
          uint32_t ebits = 0;
          if (i < live_sub) {
            const uint2 h0 = h_of(i, 0), h1 = h_of(i, 1);
            const float am = wave_row_max(fmaxf(absmax(h0), absmax(h1)));
            if (r < valid) {
              ebits = min((__float_as_uint(am) >> 23) & 0xffu, 254u);
              const int sh = 127 - static_cast<int>(ebits);
              auto qv = [&](uint32_t h) { return __builtin_amdgcn_ldexpf(bf16_bits_to_f32(h), sh); };
              uint8_t* dst = static_cast<uint8_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out;
              *reinterpret_cast<uint32_t*>(dst + hcol(0)) =
                  pack_e4m3x4(qv(h0.x & 0xffffu), qv(h0.x >> 16), qv(h0.y & 0xffffu), qv(h0.y >> 16));
              *reinterpret_cast<uint32_t*>(dst + hcol(1)) =
                  pack_e4m3x4(qv(h1.x & 0xffffu), qv(h1.x >> 16), qv(h1.y & 0xffffu), qv(h1.y >> 16));
            }
          }
          if (lg == 0) ex[r * 4 + wg] = static_cast<uint8_t>(ebits);  // 0 for rows past valid
        }
        sync_lds();
        if (tid < kBM) {
          const int q = tid;
          const int rr = (q & ~63) + (q & 15), ks = (q >> 4) & 3;
          uint32_t w = 0;
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) w |= static_cast<uint32_t>(ex[(rr + 16 * gq) * 4 + ks]) << (8 * gq);
          reinterpret_cast<uint32_t*>(p.c_scale)[static_cast<int64_t>(nt) * p.cs_rs +
                                                 static_cast<int64_t>(cur.mnat) * kBM + q] = w;
        }
      } else {
        // 1x128 group = the row's 128 columns of this tile, spread over the 4
        // waves of the group.  h (rounded to bf16) replaces the gate half of the
        // accumulators; each wave's row maxima go through LDS; the quantised
        // tile (256 rows x 128 bytes = 8 chunks) is staged in ct.
        float* rmax = reinterpret_cast<float*>(smem + kEpiOff);  // [256 rows][4 waves]
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          if (i < live_sub) {
            float m = 0.0f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const uint2 v = h_of(i, j);
              m = fmaxf(m, absmax(v));
              acc[i][j][0] = bf16_bits_to_f32(v.x & 0xffffu);
              acc[i][j][1] = bf16_bits_to_f32(v.x >> 16);
              acc[i][j][2] = bf16_bits_to_f32(v.y & 0xffffu);
              acc[i][j][3] = bf16_bits_to_f32(v.y >> 16);
            }
            m = wave_row_max(m);
            if (elg == 0) rmax[(wave_row0 + i * 16 + el16) * 4 + wg] = m;
          }
        }
        sync_lds();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = wave_row0 + i * 16 + el16;
          if (i < live_sub) {
            const f32x4 mm = *reinterpret_cast<const f32x4*>(rmax + r * 4);
            const float s = scale_from_amax(fmaxf(fmaxf(mm.x, mm.y), fmaxf(mm.z, mm.w)));
            const QuotScale qs = quot_scale(s);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const int c = wg * 2 + j;
              *reinterpret_cast<uint32_t*>(ct + r * 128 + ((c ^ (r & 7)) << 4) + elg * 4) =
                  pack_e4m3x4(quot_e4m3(acc[i][j][0], qs), quot_e4m3(acc[i][j][1], qs),
                              quot_e4m3(acc[i][j][2], qs), quot_e4m3(acc[i][j][3], qs));
            }
            if (wg == 0 && elg == 0 && r < valid) p.c_scale[static_cast<int64_t>(nt) * p.rows + row0 + r] = s;
          }
        }
        sync_lds();
        uint4 sv[4];  // reads first, then bounded stores, as in the bf16 store
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int idx = wave * 64 + eln + kThreads * u, r = idx >> 3, c = idx & 7;
          sv[u] = *reinterpret_cast<const uint4*>(ct + r * 128 + ((c ^ (r & 7)) << 4));
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int idx = wave * 64 + eln + kThreads * u, r = idx >> 3, c = idx & 7;
          store_16B<kAuxNT>(out_srd, r * p.n_out + nt * 128 + c * 16, sv[u]);
        }
        sync_lds();  // ct is the next tile's A(1) stage
      }
    }

    if (nxt.t < 0) break;
    // the claim for the tile after nxt, behind this epilogue's stores (a claim
    // issued before them would make the epilogue's first LDS store, which the
    // compiler orders after all outstanding vector memory, wait for it)
    if (kEarlyClaim && pipe && tid == 0) q_j_next = claim_start();
    if (!pipe) start_tile(nxt, buf ^ 1, gstep + k_steps);
    cur = nxt;
    buf ^= 1;
    gstep += k_steps;
  }
}
#undef HK_SLOT
#undef HK_CAP
#undef HK_SET_B
#undef HK_NROW
#undef HK_BS
#pragma clang diagnostic pop

// Packed weight layout (a load-time transform; the grouped GEMMs then read
// each K step of a weight panel as one 32 KiB block instead of 128 bytes from
// each of 256 rows 7-14 KiB apart).  For expert e, 256-row N tile nt and K
// step kt the 32 KiB block at ((e*(K/128) + kt)*(nb/256) + nt)*32 KiB holds
// the tile's sixteen 16-row MFMA fragments in operand-register order
// ("fragment-major").  The N tiles of one K step are adjacent: the narrow
// kernels, whose workgroups stream different N tiles of the same experts at
// about the same K step, read 0.8-2.7% faster than with each N tile's K steps
// adjacent (same bytes):
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
    // block order (e, kt, nt): the N tiles of one K step are adjacent
    const int nt = static_cast<int>(blk % ntile);
    const int64_t ek = blk / ntile;
    const int kt = static_cast<int>(ek % ks);
    const int64_t e = ek / ks;
    const int64_t wrow = gate_up ? nt * 128 + 32 * (R >> 6) + (R & 31) + ((R >> 5) & 1) * gate_up
                                 : static_cast<int64_t>(nt) * kBN + R;
    const uint8_t* src = w + (e * nb + wrow) * K + kt * kBK + (chunk << 4);
    *reinterpret_cast<uint4*>(out + (c << 4)) = *reinterpret_cast<const uint4*>(src);
  }
}

}  // namespace hkmoe
