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
//  * K step 128 == one scale block.  With 128x128 weight / 1x128 activation
//    block scales every MFMA of a K step covers exactly one scale block, and the
//    accumulator is kept in units of the current block's scale product:
//        u_k = u_{k-1} * (s_{k-1} / s_k) + P_k,   C = u_last * s_last,
//    so the promotion is a multiply of the accumulator *before* the MFMA that
//    reads it (no MFMA -> VALU dependency inside a K step, no partial-sum
//    registers).  Scales must be positive normal fp32 numbers.
//  * global -> LDS with buffer_load_dword{,x4} ... lds (no VGPR staging), two
//    LDS stages of 64 KiB + 1 KiB of activation scales.  Row r of a tile is
//    XOR-swizzled at 16-byte granularity (chunk c lives at c ^ ((r >> 1) & 7))
//    so ds_read_b128 operand reads of 16 consecutive rows hit distinct banks;
//    the swizzle is applied on the global side because the DMA writes lanes
//    linearly.  Activation scales are gathered by the same DMA into a
//    lane-major order (8 consecutive floats per lane).
//  * optional row gather: A row of output row p is a_gather[p] / gather_div
//    (the expert-sorted permutation), so GEMM 1 reads token rows directly and
//    no permuted copy of the activations is ever written.
//  * MFMA operands are swapped (B tile as src0, A tile as src1) so each lane
//    owns 4 consecutive output columns of one output row: 8-byte bf16 stores
//    and one activation scale per lane per 16-row sub-tile.
//  * persistent grid (one 512-thread workgroup per CU); tiles are walked in
//    groups of 8 M tiles, and workgroup ids are remapped so that the 32
//    workgroups resident on one XCD (one L2) take 32 consecutive tiles.
//  * ragged expert segments: the M-tile list comes from a device-side
//    mtile_offsets[E+1]; sub-tiles with no valid row skip loads and MFMAs.
//  * fused epilogues: bf16 store, fp32 store, or SiLU(gate)*up with either a
//    bf16 store + running |h| max (per-tensor requantisation follows) or an
//    in-tile 1x128-group requantisation to e4m3 + scales (block mode).
#pragma once

#include "common.hpp"

namespace hkmoe {

enum class Epi : int { kStoreBf16 = 0, kStoreF32 = 1, kSiluBf16 = 2, kSiluQuant = 3 };
enum class Scale : int { kTensor = 0, kBlock = 1 };

struct GemmParams {
  const uint8_t* a;            // A rows [a_rows, K] e4m3
  const int32_t* a_gather;     // optional: A row of output row p = a_gather[p] / gather_div
  const uint8_t* b;            // [E, nb, K] e4m3
  void* c;                     // [rows, n_out]: bf16, fp32 or (kSiluQuant) e4m3
  const float* a_scale;        // kTensor: [1] or null (1.0); kBlock: a_scale[r*as_rs + kb*as_ks]
  const float* b_scale;        // kTensor: [E] or null (1.0); kBlock: [E, nb/128, K/128]
  float* c_scale;              // kSiluQuant: group scales, transposed [n_out/128, rows]
  const int32_t* offsets;      // [E+1] row offsets; nullptr = dense (one segment of `rows`)
  const int32_t* mtile_offsets;// [E+1] M-tile offsets; nullptr = dense
  float* amax;                 // kSiluBf16: running max |h| (uint-ordered), may be null
  int64_t rows;                // output rows (dense: M)
  int64_t a_rows;              // rows addressable through `a` (buffer bound)
  int64_t as_rs, as_ks;        // activation scale strides (row, K block)
  int32_t gather_div;
  int32_t num_experts;
  int32_t K;
  int32_t nb;                  // B rows per expert (N, or 2I for the fused gate/up GEMM)
  int32_t n_out;               // output columns (N, or I)
  int32_t n_tiles;             // N tiles per M tile
};

constexpr int kBM = 256, kBN = 256, kBK = 128;
constexpr int kThreads = 512;
constexpr int kTileBytes = kBM * kBK;                    // 32 KiB per operand
constexpr int kScaleBytes = kBM * 4;                     // activation scales of one K step
constexpr int kStageBytes = 2 * kTileBytes + kScaleBytes;
constexpr int kMaxKBlocks = 128;                         // K <= 16384
constexpr int kBsBytes = 2 * kMaxKBlocks * 4;            // weight scales of one tile
constexpr int kRedBytes = 4 * kBM * 4;                   // epilogue cross-wave row max
constexpr int kLdsBytes = 2 * kStageBytes + kBsBytes + kRedBytes;
constexpr int kGroupM = 8;

static_assert(kLdsBytes <= 160 * 1024, "LDS budget");

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

// Position of tile row r in the lane-major activation-scale layout: the lane
// with l16 = r % 16 of wave-row r / 128 reads its 8 sub-tile scales as 8
// consecutive floats.
__device__ __forceinline__ int scale_slot_row(int slot) {
  const int wm = slot >> 7, w = slot & 127;
  return wm * 128 + (w & 7) * 16 + (w >> 3);
}

template <Epi EPI, Scale SC>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_persistent(GemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  float* bs_lds = reinterpret_cast<float*>(smem + 2 * kStageBytes);       // [2][kblocks]
  float* red_lds = reinterpret_cast<float*>(smem + 2 * kStageBytes + kBsBytes);  // [4][256]

  constexpr bool kBlockSc = (SC == Scale::kBlock);
  constexpr bool kSilu = (EPI == Epi::kSiluBf16 || EPI == Epi::kSiluQuant);

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

  const i32x4 a_srd = make_srd(p.a, static_cast<uint32_t>(min<int64_t>(p.a_rows * p.K, 0xffffffffll)));

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

    const uint8_t* b_expert = p.b + static_cast<int64_t>(e) * p.nb * p.K;
    const i32x4 b_srd = make_srd(b_expert, static_cast<uint32_t>(p.nb) * p.K);

    // B rows held by this tile: LDS row `r` maps to weight row b_row(r).
    // kSilu: quarter q (64 rows) = 32 gate rows then the 32 matching up rows.
    auto b_row = [&](int r) -> int {
      if constexpr (kSilu) {
        const int q = r >> 6, w = r & 63;
        const int col = nt * 128 + q * 32 + (w & 31);
        return (w < 32) ? col : (p.n_out + col);
      } else {
        return nt * kBN + r;
      }
    };
    auto a_row_of = [&](int r) -> int64_t {  // A row feeding output row row0 + r
      const int rr = row0 + min(r, valid - 1);
      return p.a_gather ? static_cast<int64_t>(p.a_gather[rr] / p.gather_div) : rr;
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
      a_voff[i] = static_cast<int>(a_row_of(r) * p.K) + c * 16;
      a_live[i] = ((grp8 * 8) & ~15) < valid;
      b_voff[i] = b_row(r) * p.K + c * 16;
    }
    // activation scales: waves 0..3 each gather 64 of the tile's 256 rows
    int as_voff = 0;
    if constexpr (kBlockSc) {
      const int slot = (wave & 3) * 64 + lane;
      as_voff = static_cast<int>(a_row_of(scale_slot_row(slot)) * p.as_rs) * 4;
    }
    const i32x4 as_srd = kBlockSc ? make_srd(p.a_scale, 0xffffffffu) : i32x4{0, 0, 0, 0};

    auto issue_stage = [&](int kt, int stage) {
      uint8_t* sa = smem + stage * kStageBytes;
      uint8_t* sb = sa + kTileBytes;
      const int koff = kt * kBK;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int grp8 = i * 8 + wave;
        if (a_live[i]) load_lds_16B(a_srd, sa + grp8 * 1024, a_voff[i] + koff);
        load_lds_16B(b_srd, sb + grp8 * 1024, b_voff[i] + koff);
      }
      if constexpr (kBlockSc) {
        if (wave < 4)
          load_lds_4B(as_srd, sb + kTileBytes + wave * 256,
                      as_voff + static_cast<int>(kt * p.as_ks) * 4);
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

    __syncthreads();  // previous tile's readers are done with every LDS buffer
    if constexpr (kBlockSc) {
      // weight scales of this tile for every K block: [2][kblocks]
      const int kblocks = k_iters;
      const float* bs = p.b_scale + static_cast<int64_t>(e) * (p.nb / kGroup) * kblocks;
      const int nb0 = kSilu ? nt : 2 * nt;                       // gate / first n block
      const int nb1 = kSilu ? (p.n_out / kGroup + nt) : 2 * nt + 1;  // up / second n block
      for (int t = tid; t < 2 * kblocks; t += kThreads) {
        const int h = t / kblocks, kb = t - h * kblocks;
        bs_lds[t] = bs[(h ? nb1 : nb0) * kblocks + kb];
      }
    }
    issue_stage(0, 0);

    // which weight-scale half feeds n sub-tile j of this wave
    // kSilu: j = 0,1 gate, 2,3 up.  Plain: the wave's 64 columns sit in n block
    // (wn * 64) / 128 of the tile.
    float s_prev[8][2];

    for (int kt = 0; kt < k_iters; ++kt) {
      const int stage = kt & 1;
      wait_vmem_all();
      __syncthreads();
      if (kt + 1 < k_iters) issue_stage(kt + 1, stage ^ 1);

      const uint8_t* sa = smem + stage * kStageBytes;
      const uint8_t* sb = sa + kTileBytes;

      i32x8 bf[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = read_frag(sb, wn * 64 + j * 16 + l16, lg);

      float r_fac[8][2];
      if constexpr (kBlockSc) {
        const float* sc = reinterpret_cast<const float*>(sb + kTileBytes) + wm * 128 + l16 * 8;
        const f32x4 s_lo = *reinterpret_cast<const f32x4*>(sc);
        const f32x4 s_hi = *reinterpret_cast<const f32x4*>(sc + 4);
        const float sa_v[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
        float sb_v[2];
        if constexpr (kSilu) {
          sb_v[0] = bs_lds[kt];
          sb_v[1] = bs_lds[k_iters + kt];
        } else {
          sb_v[0] = sb_v[1] = bs_lds[(wn >> 1) * k_iters + kt];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float s_cur = sa_v[i] * sb_v[h];
            r_fac[i][h] = (kt == 0) ? 1.0f : s_prev[i][h] * __builtin_amdgcn_rcpf(s_cur);
            s_prev[i][h] = s_cur;
          }
      }

      i32x8 af_next = read_frag(sa, wave_row0 + l16, lg);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (i < live_sub) {
          const i32x8 af = af_next;
          if (i + 1 < 8 && i + 1 < live_sub) af_next = read_frag(sa, wave_row0 + (i + 1) * 16 + l16, lg);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            if constexpr (kBlockSc) acc[i][j] *= r_fac[i][kSilu ? (j >> 1) : 0];
            acc[i][j] = mfma_e4m3_16x16x128(bf[j], af, acc[i][j]);
          }
        }
      }
    }

    // ---- epilogue ----------------------------------------------------------
    // fold the last block's scale product (block) or the per-tensor scales back in
    float fac[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (kBlockSc)
          fac[i][h] = s_prev[i][h];
        else
          fac[i][h] = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[e] : 1.0f);
      }

    if constexpr (kSilu) {
      // h = bf16(silu(g) * u); lane holds gate/up for columns col..col+3 of row r
      uint32_t hb[8][2][4];
      float row_max[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        row_max[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const float gv = acc[i][j][q] * fac[i][0];
            const float uv = acc[i][j + 2][q] * fac[i][1];
            hb[i][j][q] = bf16_rne_bits(silu(gv) * uv);
            row_max[i] = fmaxf(row_max[i], fabsf(bf16_bits_to_f32(hb[i][j][q])));
          }
      }
      if constexpr (EPI == Epi::kSiluBf16) {
        float local_max = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = wave_row0 + i * 16 + l16;
          if (i < live_sub && r < valid) {
            local_max = fmaxf(local_max, row_max[i]);
            uint16_t* crow = static_cast<uint16_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const int col = nt * 128 + wn * 32 + j * 16 + lg * 4;
              uint2 v;
              v.x = hb[i][j][0] | (hb[i][j][1] << 16);
              v.y = hb[i][j][2] | (hb[i][j][3] << 16);
              *reinterpret_cast<uint2*>(crow + col) = v;
            }
          }
        }
        const float m = wave_max(local_max);
        if (lane == 0 && p.amax != nullptr)
          atomicMax(reinterpret_cast<unsigned int*>(p.amax), __float_as_uint(m));
      } else {
        // 1x128 group requantisation: the tile's 128 intermediate columns of a
        // row are one group, spread over 4 lane groups x 4 waves.
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float m = row_max[i];
          m = fmaxf(m, __shfl_xor(m, 16, 64));
          m = fmaxf(m, __shfl_xor(m, 32, 64));
          if (lg == 0) red_lds[wn * kBM + wave_row0 + i * 16 + l16] = m;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int r = wave_row0 + i * 16 + l16;
          if (i < live_sub && r < valid) {
            const float amax = fmaxf(fmaxf(red_lds[r], red_lds[kBM + r]),
                                     fmaxf(red_lds[2 * kBM + r], red_lds[3 * kBM + r]));
            const float s = scale_from_amax(amax);
            uint8_t* crow = static_cast<uint8_t*>(p.c) + static_cast<int64_t>(row0 + r) * p.n_out;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
              const int col = nt * 128 + wn * 32 + j * 16 + lg * 4;
              uint32_t qv = 0;
#pragma unroll
              for (int q = 0; q < 4; ++q) qv |= f32_to_e4m3(bf16_bits_to_f32(hb[i][j][q]) / s) << (8 * q);
              *reinterpret_cast<uint32_t*>(crow + col) = qv;
            }
            if (wn == 0 && lg == 0) p.c_scale[static_cast<int64_t>(nt) * p.rows + row0 + r] = s;
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int r = wave_row0 + i * 16 + l16;
        if (i < live_sub && r < valid) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float f = fac[i][0];
            const int col = nt * kBN + wn * 64 + j * 16 + lg * 4;
            const int64_t off = static_cast<int64_t>(row0 + r) * p.n_out + col;
            if constexpr (EPI == Epi::kStoreF32) {
              float4 v;
              v.x = acc[i][j][0] * f; v.y = acc[i][j][1] * f;
              v.z = acc[i][j][2] * f; v.w = acc[i][j][3] * f;
              *reinterpret_cast<float4*>(static_cast<float*>(p.c) + off) = v;
            } else {
              uint2 v;
              v.x = pack_bf16x2(acc[i][j][0] * f, acc[i][j][1] * f);
              v.y = pack_bf16x2(acc[i][j][2] * f, acc[i][j][3] * f);
              *reinterpret_cast<uint2*>(static_cast<uint16_t*>(p.c) + off) = v;
            }
          }
        }
      }
    }
  }
}

}  // namespace hkmoe
