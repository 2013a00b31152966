// Persistent FP8 (e4m3 x e4m3 -> fp32) GEMM core for gfx950, shared by the
// dense GEMM and both grouped (per-expert) MoE GEMMs.
//
// C[m, n] = sum_k A[m, k] * B[n, k]   ("TN": both operands K-contiguous), the
// convention of the reference's mma_ABt kernels
// (kernels/cdna4/gemm/mxfp8/MXFP8_4wave/4_wave.cu:77-292, cdna3
// 256_256_64_32.cpp:32-200).  Design (all new, CDNA4-first):
//
//  * block tile 256 (rows of A) x 256 (rows of B) x 128 (K), 8 waves as 2 x 4;
//    each wave owns a 128 x 64 sub-tile = 8 x 4 MFMA 16x16x128 tiles.
//  * K step 128 == one scale block, so with 128x128 / 1x128 block scales a
//    single MFMA yields exactly one block's partial sum; it is promoted into the
//    fp32 accumulator with one FMA per element (no extra partial registers).
//  * global -> LDS with buffer_load_dwordx4 ... lds (no VGPR staging), two LDS
//    stages of 64 KiB.  The LDS image of a row is XOR-swizzled at 16-byte
//    granularity (chunk c of row r lives at c ^ ((r >> 1) & 7)) so that the
//    ds_read_b128 operand reads of 16 consecutive rows hit distinct banks; the
//    swizzle is applied on the global side because the DMA writes lanes
//    linearly.
//  * MFMA operands are swapped (B tile as src0, A tile as src1) so each lane
//    ends up owning 4 consecutive output columns of one output row: 8-byte
//    bf16 stores and one activation scale per lane per 16-row sub-tile.
//  * persistent grid (one 512-thread workgroup per CU); tiles are walked in
//    groups of 8 M-tiles, and workgroup ids are remapped so that the 32
//    workgroups resident on one XCD (one L2) take 32 consecutive tiles.
//  * ragged expert segments: the M-tile list is given by a device-side
//    mtile_offsets[E+1]; sub-tiles with no valid row skip their loads and MFMAs.
#pragma once

#include "common.hpp"

namespace hkmoe {

enum class Epi : int { kStoreBf16 = 0, kStoreF32 = 1, kSiluBf16 = 2 };
enum class Scale : int { kTensor = 0, kBlock = 1 };

struct GemmParams {
  const uint8_t* a;            // [rows, K] e4m3 (rows expert-contiguous)
  const uint8_t* b;            // [E, nb, K] e4m3
  void* c;                     // [rows, n_out] (bf16 or fp32)
  const float* a_scale;        // kTensor: [1] or null (1.0); kBlock: [K/128, a_scale_ld]
  const float* b_scale;        // kTensor: [E] or null (1.0); kBlock: [E, nb/128, K/128]
  const int32_t* offsets;      // [E+1] row offsets; nullptr = dense (one segment of `rows`)
  const int32_t* mtile_offsets;// [E+1] M-tile offsets; nullptr = dense
  float* amax;                 // kSiluBf16 + kTensor: running max |h| (uint-ordered), else null
  int64_t rows;                // dense: M
  int64_t a_scale_ld;          // leading dimension of the transposed activation scales
  int32_t num_experts;
  int32_t K;
  int32_t nb;                  // B rows per expert (N, or 2I for the fused gate/up GEMM)
  int32_t n_out;               // output columns (N, or I)
  int32_t n_tiles;             // N tiles per M tile
};

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kThreads = 512;
constexpr int kStageBytes = (kBM + kBN) * kBK;  // 64 KiB
constexpr int kLdsBytes = 2 * kStageBytes;      // 128 KiB
constexpr int kGroupM = 8;

__device__ __forceinline__ int swz_chunk(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Read one 16x128 operand fragment (32 bytes per lane) from a swizzled tile.
__device__ __forceinline__ i32x8 read_frag(const uint8_t* tile, int row, int half) {
  const int c0 = swz_chunk(row, 2 * half), c1 = swz_chunk(row, 2 * half + 1);
  const i32x4 lo = *reinterpret_cast<const i32x4*>(tile + row * kBK + c0 * 16);
  const i32x4 hi = *reinterpret_cast<const i32x4*>(tile + row * kBK + c1 * 16);
  i32x8 r;
  r.s0 = lo.x; r.s1 = lo.y; r.s2 = lo.z; r.s3 = lo.w;
  r.s4 = hi.x; r.s5 = hi.y; r.s6 = hi.z; r.s7 = hi.w;
  return r;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

template <Epi EPI, Scale SC>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_persistent(GemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int wm = wave >> 2;   // 0..1  -> 128-row half of the tile
  const int wn = wave & 3;    // 0..3  -> 64-column quarter of the tile
  const int l16 = lane & 15;
  const int lg = lane >> 4;   // 0..3

  const bool dense = (p.offsets == nullptr);
  const int total_mtiles = dense ? static_cast<int>((p.rows + kBM - 1) / kBM)
                                 : __builtin_amdgcn_readfirstlane(p.mtile_offsets[p.num_experts]);
  const int total_tiles = total_mtiles * p.n_tiles;
  const int k_iters = p.K / kBK;

  // XCD-aware virtual id: workgroups are dispatched round-robin over 8 XCDs,
  // so blockIdx % 8 is the XCD; give each XCD a contiguous run of ids.
  const int g = gridDim.x;
  const int per_xcd = g >> 3;
  const int vid = (g & 7) == 0 ? (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3) : blockIdx.x;

  for (int tile = vid; tile < total_tiles; tile += g) {
    // ---- tile -> (M tile, N tile), grouped by kGroupM M tiles -------------
    const int per_group = kGroupM * p.n_tiles;
    const int grp = tile / per_group;
    const int within = tile - grp * per_group;
    const int gm_size = min(kGroupM, total_mtiles - grp * kGroupM);
    const int mt_glob = grp * kGroupM + within % gm_size;
    const int nt = within / gm_size;

    // ---- M tile -> expert segment ----------------------------------------
    int e = 0, row0 = 0, valid = 0;
    if (dense) {
      row0 = mt_glob * kBM;
      valid = static_cast<int>(min<int64_t>(kBM, p.rows - row0));
    } else {
      int lo = 0, hi = p.num_experts;  // largest e with mtile_offsets[e] <= mt_glob
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (p.mtile_offsets[mid] <= mt_glob) lo = mid; else hi = mid;
      }
      e = lo;
      const int seg0 = p.offsets[e], seg1 = p.offsets[e + 1];
      row0 = seg0 + (mt_glob - p.mtile_offsets[e]) * kBM;
      valid = min(kBM, seg1 - row0);
    }
    e = __builtin_amdgcn_readfirstlane(e);
    row0 = __builtin_amdgcn_readfirstlane(row0);
    valid = __builtin_amdgcn_readfirstlane(valid);

    // ---- descriptors -----------------------------------------------------
    const uint8_t* a_base = p.a + static_cast<int64_t>(row0) * p.K;
    const i32x4 a_srd = make_srd(a_base, static_cast<uint32_t>(valid) * p.K);
    const uint8_t* b_expert = p.b + static_cast<int64_t>(e) * p.nb * p.K;
    const i32x4 b_srd = make_srd(b_expert, static_cast<uint32_t>(p.nb) * p.K);

    // B rows held by this tile: row `r` of the LDS tile maps to weight row brow(r)
    // kSilu: quarter q (64 rows) = 32 gate rows then the 32 matching up rows.
    auto b_row = [&](int r) -> int {
      if constexpr (EPI == Epi::kSiluBf16) {
        const int q = r >> 6, w = r & 63;
        const int col = nt * 128 + q * 32 + (w & 31);
        return (w < 32) ? col : (p.n_out + col);
      } else {
        return nt * kBN + r;
      }
    };

    // Each wave issues 4 A + 4 B wave-loads (8 rows x 128 B each) per K step.
    // A row groups whose 16-row sub-tile has no valid row are skipped; rows past
    // `valid` inside a live sub-tile read the last valid row (results dropped).
    const int ld_row_in_grp = lane >> 3;   // 0..7
    const int ld_pchunk = lane & 7;        // physical 16-byte chunk in LDS
    int a_voff[4], b_voff[4];
    bool a_live[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int grp8 = i * 8 + wave;       // 0..31 -> rows 8*grp8 .. +7
      const int r = grp8 * 8 + ld_row_in_grp;
      const int c = swz_chunk(r, ld_pchunk);
      const int ra = min(r, valid - 1);
      a_voff[i] = ra * p.K + c * 16;
      a_live[i] = ((grp8 * 8) & ~15) < valid;
      b_voff[i] = b_row(r) * p.K + c * 16;
    }

    auto issue_stage = [&](int kt, int stage) {
      uint8_t* sa = smem + stage * kStageBytes;
      uint8_t* sb = sa + kBM * kBK;
      const int koff = kt * kBK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int grp8 = i * 8 + wave;
        if (a_live[i]) load_lds_16B(a_srd, sa + grp8 * 1024, a_voff[i] + koff);
        load_lds_16B(b_srd, sb + grp8 * 1024, b_voff[i] + koff);
      }
    };

    // ---- accumulators -----------------------------------------------------
    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // number of live 16-row sub-tiles for this wave's 128-row half
    const int wave_row0 = wm * 128;
    const int live_sub = max(0, min(8, (valid - wave_row0 + 15) >> 4));

    // block-scale bookkeeping
    int sb_idx[4];
    const float* a_sc = nullptr;
    if constexpr (SC == Scale::kBlock) {
      const int kblocks = p.K / kGroup;
      const float* bs = p.b_scale + static_cast<int64_t>(e) * (p.nb / kGroup) * kblocks;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int brow = b_row(wn * 64 + j * 16);
        sb_idx[j] = (brow / kGroup) * kblocks;
      }
      (void)bs;
      a_sc = p.a_scale;
    }

    __syncthreads();  // previous tile's readers are done with both stages
    issue_stage(0, 0);

    for (int kt = 0; kt < k_iters; ++kt) {
      const int stage = kt & 1;
      wait_vmem_all();
      __syncthreads();
      if (kt + 1 < k_iters) issue_stage(kt + 1, stage ^ 1);

      const uint8_t* sa = smem + stage * kStageBytes;
      const uint8_t* sb = sa + kBM * kBK;

      i32x8 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = read_frag(sb, wn * 64 + j * 16 + l16, lg);

      float sbv[4];
      if constexpr (SC == Scale::kBlock) {
        const float* bs = p.b_scale + static_cast<int64_t>(e) * (p.nb / kGroup) * (p.K / kGroup);
#pragma unroll
        for (int j = 0; j < 4; ++j) sbv[j] = bs[sb_idx[j] + kt];
      }

#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i < live_sub) {
          const int ar = wave_row0 + i * 16 + l16;
          const i32x8 af = read_frag(sa, ar, lg);
          if constexpr (SC == Scale::kBlock) {
            const int arow = min(ar, valid - 1);
            const float sav = a_sc[static_cast<int64_t>(kt) * p.a_scale_ld + row0 + arow];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const f32x4 part = mfma_e4m3_16x16x128(bf[j], af, f32x4{0.f, 0.f, 0.f, 0.f});
              const float s = sav * sbv[j];
              acc[i][j] += part * s;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = mfma_e4m3_16x16x128(bf[j], af, acc[i][j]);
          }
        }
      }
    }

    // ---- epilogue ----------------------------------------------------------
    float factor = 1.0f;
    if constexpr (SC == Scale::kTensor)
      factor = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[e] : 1.0f);

    if constexpr (EPI == Epi::kSiluBf16) {
      float local_max = 0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave_row0 + i * 16 + l16;
        if (i < live_sub && r < valid) {
          uint16_t* crow = static_cast<uint16_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const int col = nt * 128 + wn * 32 + j * 16 + lg * 4;
            uint32_t hb[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float gv = acc[i][j][q] * factor;
              const float uv = acc[i][j + 2][q] * factor;
              hb[q] = bf16_rne_bits(silu(gv) * uv);
              local_max = fmaxf(local_max, fabsf(bf16_bits_to_f32(hb[q])));
            }
            uint2 v;
            v.x = hb[0] | (hb[1] << 16);
            v.y = hb[2] | (hb[3] << 16);
            *reinterpret_cast<uint2*>(crow + col) = v;
          }
        }
      }
      if constexpr (SC == Scale::kTensor) {
        const float m = wave_max(local_max);
        if (lane == 0 && p.amax != nullptr)
          atomicMax(reinterpret_cast<unsigned int*>(p.amax), __float_as_uint(m));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave_row0 + i * 16 + l16;
        if (i < live_sub && r < valid) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int col = nt * kBN + wn * 64 + j * 16 + lg * 4;
            const int64_t off = static_cast<int64_t>(row0 + r) * p.n_out + col;
            if constexpr (EPI == Epi::kStoreF32) {
              float4 v;
              v.x = acc[i][j][0] * factor; v.y = acc[i][j][1] * factor;
              v.z = acc[i][j][2] * factor; v.w = acc[i][j][3] * factor;
              *reinterpret_cast<float4*>(static_cast<float*>(p.c) + off) = v;
            } else {
              uint2 v;
              v.x = pack_bf16x2(acc[i][j][0] * factor, acc[i][j][1] * factor);
              v.y = pack_bf16x2(acc[i][j][2] * factor, acc[i][j][3] * factor);
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.c) + off) = v;
            }
          }
        }
      }
    }
  }
}

}  // namespace hkmoe
