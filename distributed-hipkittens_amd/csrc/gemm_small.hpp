// Dense FP8 GEMM for problems with few 256x256 tiles (fewer than two per CU):
// C[M,N] = (sa*sb) * A[M,K] . B[N,K]^T with per-tensor scales, bf16 or fp32 C.
//
// 128x128 output tiles, one non-persistent workgroup of 4 waves per tile, one
// wave per SIMD, each wave 64x64 outputs: 4x4 v_mfma_f32_16x16x128_f8f6f4 per
// K step, or (M32) 2x2 blocks of 32x32 outputs, each two
// v_mfma_f32_32x32x64_f8f6f4 (the two 64-byte halves of the K step).
// With one wave per SIMD there is no ping-pong partner: the wave overlaps its
// own LDS fragment reads of step kt+1 with its MFMAs of step kt (two register
// sets of fragments), and a 4-deep LDS ring fed by buffer->LDS DMA keeps three
// K steps (96 KiB per CU) in flight (a fifth stage measured slower).  The 2048^3 GEMM (config 1) is 256 such
// tiles, one per CU, where the 256x256 kernel has 64.
#pragma once

#include "gemm_fp8.hpp"

namespace hkmoe {

constexpr int kSmTile = 128;                         // output tile edge
constexpr int kSmThreads = 256;                      // 4 waves
constexpr int kSmStages = 4;                         // LDS ring depth (K steps)
constexpr int kSmAhead = kSmStages - 1;              // K steps in flight beyond the current one
constexpr int kSmOperandBytes = kSmTile * kBK;       // 16 KiB per operand per step
constexpr int kSmStageBytes = 2 * kSmOperandBytes;   // A then B
constexpr int kSmLdsBytes = kSmStages * kSmStageBytes;  // 128 KiB
static_assert(kSmLdsBytes <= 160 * 1024, "LDS budget");
static_assert(kSmTile * kSmTile * 2 <= kSmStageBytes, "the bf16 output tile is staged in one stage");

struct SmallGemmParams {
  const uint8_t* a;        // [M, K] e4m3
  const uint8_t* b;        // [N, K] e4m3
  void* c;                 // [M, N] bf16 or fp32
  const float* a_scale;    // optional per-tensor scales
  const float* b_scale;
  int32_t m, n, k;
  uint32_t a_bytes, b_bytes;  // buffer bounds (min(rows * K, 2^32 - 1))
  int32_t m_tiles, n_tiles;   // 128-row / 128-column tiles
  int32_t nbn;                // tile blocks per block row: ceil(n_tiles / 8)
};

// vmcnt wait leaving the newest n_newer stages (8 loads each) of this wave in
// flight, then a barrier: every wave's loads of the older stages are in LDS.
__device__ __forceinline__ void small_wait_stage(int n_newer) {
  if (n_newer >= 3) asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else if (n_newer == 2) asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else if (n_newer == 1) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
static_assert(kSmAhead <= 4, "small_wait_stage covers at most 3 newer stages");

template <bool F32OUT, bool M32>
__global__ __launch_bounds__(kSmThreads, 1) void gemm_fp8_small(SmallGemmParams p) {
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15, lg = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;  // the wave's 64x64 quarter
  const int fx = swz(l16);

  // Tile of this workgroup.  Workgroups are dispatched round-robin over the 8
  // XCDs (blockIdx % 8), so each XCD gets a contiguous run of virtual ids, and
  // a run of 32 ids is a block of 4 (M) x 8 (N) tiles sharing A rows and B
  // columns in that XCD's L2.  The grid is a whole number of blocks; ids past
  // the tile grid exit.
  const int g = gridDim.x;
  const int vid = (g & 7) == 0 ? (blockIdx.x & 7) * (g >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int blk = vid >> 5, sl = vid & 31;
  const int mt = (blk / p.nbn) * 4 + (sl & 3), nt = (blk % p.nbn) * 8 + (sl >> 2);
  if (mt >= p.m_tiles || nt >= p.n_tiles) return;
  const int m0 = mt * kSmTile, n0 = nt * kSmTile;
  const int k_steps = p.k / kBK;

  // DMA: instruction i of wave w fills LDS rows 32i + 8w + lane/8 of an operand
  // tile; the lane fetches logical chunk (lane & 7) ^ swz(row), which lands
  // swizzled.  A rows past M repeat row M-1 (never stored).
  const int ld_row = 8 * wave + (lane >> 3);
  const int ld_chunk = (lane & 7) ^ swz(ld_row);
  const i32x4 a_srd = make_srd(p.a, p.a_bytes);
  const i32x4 b_srd = make_srd(p.b, p.b_bytes);
  int a_voff[4], b_voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ra = min(m0 + 32 * i + ld_row, p.m - 1);
    a_voff[i] = buf_off(ra, p.k, ld_chunk * 16);
    b_voff[i] = buf_off(n0 + 32 * i + ld_row, p.k, ld_chunk * 16);
  }
  auto issue = [&](int kt) __attribute__((always_inline)) {
    uint8_t* st = smem + (kt % kSmStages) * kSmStageBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) load_lds_16B(a_srd, st + (32 * i + 8 * wave) * kBK, a_voff[i], kt * kBK);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      load_lds_16B(b_srd, st + kSmOperandBytes + (32 * i + 8 * wave) * kBK, b_voff[i], kt * kBK);
  };
  // The wave's fragments of step kt.  16x16x128: A sub-tiles (rows 64wm + 16i
  // + l16) and B fragments (columns 64wn + 16j + l16), K bytes 32lg .. +31.
  // M32: fragment 2b + h is 32-row block b (rows 64wm + 32b + l32 of A, 64wn +
  // 32b + l32 of B) and K half h: bytes 64h + 32g .. +31 (g = lane / 32), i.e.
  // the 32-byte chunk pair 2h + g of the row; the rows of a block start at a
  // multiple of 32, so the swizzle of row l32 is the lane constant f32.
  const int l32 = lane & 31, g32 = lane >> 5;
  const int f32 = swz(l32);
  auto read = [&](int kt, i32x8 (&af)[4], i32x8 (&bf)[4]) __attribute__((always_inline)) {
    const uint8_t* st = smem + (kt % kSmStages) * kSmStageBytes;
    if constexpr (M32) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        af[f] = read_frag(st, 64 * wm + 32 * (f >> 1) + l32, 2 * (f & 1) + g32, f32);
        bf[f] = read_frag(st + kSmOperandBytes, 64 * wn + 32 * (f >> 1) + l32, 2 * (f & 1) + g32, f32);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) af[i] = read_frag(st, 64 * wm + 16 * i + l16, lg, fx);
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = read_frag(st + kSmOperandBytes, 64 * wn + 16 * j + l16, lg, fx);
    }
  };

  // accumulators: 16x16x128: acc[i][j] (4 values); M32: acc32[bi][bj] (16 values)
  f32x4 acc[4][4];
  f32x16 acc32[2][2];
  if constexpr (M32) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc32[i][j][r] = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  auto mma = [&](const i32x8 (&af)[4], const i32x8 (&bf)[4]) __attribute__((always_inline)) {
    if constexpr (M32) {
      // both K halves of the four blocks; a block's second MFMA is issued three
      // MFMAs after its first
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc32[i][j] = mfma_e4m3_32x32x64(bf[2 * j + h], af[2 * i + h], acc32[i][j]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma_e4m3_16x16x128(bf[j], af[i], acc[i][j]);
    }
  };

  // Prologue: steps 0 .. kSmAhead-1 in flight, step 0's fragments in registers.
  const int pre = min(kSmAhead, k_steps);
  for (int kt = 0; kt < pre; ++kt) issue(kt);
  small_wait_stage(pre - 1);
  i32x8 af0[4], bf0[4], af1[4], bf1[4];
  read(0, af0, bf0);

  // Step kt: DMA of step kt+kSmAhead into the slot of step kt-1 (read in
  // iteration kt-2, complete at iteration kt-1's barrier); wait for step kt+1;
  // read its fragments into the other register set while the MFMAs of step kt
  // run.
  auto step = [&](int kt, i32x8 (&ca)[4], i32x8 (&cb)[4], i32x8 (&na)[4], i32x8 (&nb)[4])
      __attribute__((always_inline)) {
    if (kt + kSmAhead < k_steps) issue(kt + kSmAhead);
    if (kt + 1 < k_steps) {
      small_wait_stage(min(kSmAhead - 1, k_steps - 1 - (kt + 1)));
      read(kt + 1, na, nb);
    }
    // the reads stay ahead of the MFMAs (left behind them, the next step's
    // barrier, which waits for them, would expose their whole latency)
    __builtin_amdgcn_sched_barrier(0);
    mma(ca, cb);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Steady state, straight-line: every step issues a load and leaves kSmAhead-1
  // newer steps in flight.  (Written with the tail's conditions, the two
  // register sets got merged into one, which put each step's reads right
  // before its own MFMAs.)
  auto step_full = [&](int kt, i32x8 (&ca)[4], i32x8 (&cb)[4], i32x8 (&na)[4], i32x8 (&nb)[4])
      __attribute__((always_inline)) {
    issue(kt + kSmAhead);
    small_wait_stage(kSmAhead - 1);
    read(kt + 1, na, nb);
    __builtin_amdgcn_sched_barrier(0);
    mma(ca, cb);
    __builtin_amdgcn_sched_barrier(0);
  };
  int kt = 0;
  for (; kt + 1 + kSmAhead < k_steps; kt += 2) {
    step_full(kt, af0, bf0, af1, bf1);
    step_full(kt + 1, af1, bf1, af0, bf0);
  }
  for (; kt + 1 < k_steps; kt += 2) {
    step(kt, af0, bf0, af1, bf1);
    step(kt + 1, af1, bf1, af0, bf0);
  }
  if (kt < k_steps) step(kt, af0, bf0, af1, bf1);

  // ---- epilogue: lane holds row 64wm + 16i + l16, columns 64wn + 16j + 4lg .. +3
  // (M32: row 64wm + 32bi + l32, columns 64wn + 32bj + 8q + 4g32 .. +3 in
  // registers 4q .. 4q+3 of acc32[bi][bj])
  const float tens = (p.a_scale ? p.a_scale[0] : 1.0f) * (p.b_scale ? p.b_scale[0] : 1.0f);
  if constexpr (M32 && F32OUT) {
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const int r = m0 + 64 * wm + 32 * bi + l32;
      if (r < p.m) {
#pragma unroll
        for (int bj = 0; bj < 2; ++bj) {
          float* dst = static_cast<float*>(p.c) + static_cast<int64_t>(r) * p.n + n0 + 64 * wn + 32 * bj + 4 * g32;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4*>(dst + 8 * q) =
                float4{acc32[bi][bj][4 * q] * tens, acc32[bi][bj][4 * q + 1] * tens,
                       acc32[bi][bj][4 * q + 2] * tens, acc32[bi][bj][4 * q + 3] * tens};
        }
      }
    }
  } else if constexpr (M32) {
    // staged as below: row r, 16-byte chunk c = 8wn + 4bj + q, 8-byte half g32
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int bi = 0; bi < 2; ++bi) {
      const int r = 64 * wm + 32 * bi + l32;
#pragma unroll
      for (int bj = 0; bj < 2; ++bj)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c = 8 * wn + 4 * bj + q;
          uint2 v;
          v.x = pack_bf16x2(acc32[bi][bj][4 * q] * tens, acc32[bi][bj][4 * q + 1] * tens);
          v.y = pack_bf16x2(acc32[bi][bj][4 * q + 2] * tens, acc32[bi][bj][4 * q + 3] * tens);
          *reinterpret_cast<uint2*>(smem + r * 256 + ((c ^ (r & 15)) << 4) + g32 * 8) = v;
        }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = tid + kSmThreads * u, r = idx >> 4, c = idx & 15;
      if (m0 + r < p.m) {
        const uint4 v = *reinterpret_cast<const uint4*>(smem + r * 256 + ((c ^ (r & 15)) << 4));
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.c) + static_cast<int64_t>(m0 + r) * p.n + n0 + c * 8) = v;
      }
    }
  } else if constexpr (F32OUT) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m0 + 64 * wm + 16 * i + l16;
      if (r < p.m) {
        float* dst = static_cast<float*>(p.c) + static_cast<int64_t>(r) * p.n + n0 + 64 * wn + 4 * lg;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<float4*>(dst + 16 * j) =
              float4{acc[i][j][0] * tens, acc[i][j][1] * tens, acc[i][j][2] * tens, acc[i][j][3] * tens};
      }
    }
  } else {
    // staged in LDS (rows of 256 bytes = 16 chunks, chunk c of row r at slot
    // c ^ (r & 15)) and stored as 16-byte chunks covering whole rows
    __syncthreads();  // every wave is done with the ring
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 64 * wm + 16 * i + l16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int c = 8 * wn + 2 * j + (lg >> 1);
        uint2 v;
        v.x = pack_bf16x2(acc[i][j][0] * tens, acc[i][j][1] * tens);
        v.y = pack_bf16x2(acc[i][j][2] * tens, acc[i][j][3] * tens);
        *reinterpret_cast<uint2*>(smem + r * 256 + ((c ^ (r & 15)) << 4) + (lg & 1) * 8) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int idx = tid + kSmThreads * u, r = idx >> 4, c = idx & 15;
      if (m0 + r < p.m) {
        const uint4 v = *reinterpret_cast<const uint4*>(smem + r * 256 + ((c ^ (r & 15)) << 4));
        *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.c) + static_cast<int64_t>(m0 + r) * p.n + n0 + c * 8) = v;
      }
    }
  }
}

}  // namespace hkmoe
