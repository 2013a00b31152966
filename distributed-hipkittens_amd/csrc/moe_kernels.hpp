// Routing, scatter (permute), requantisation, combine and quantiser kernels
// for the gfx950 FP8 MoE path.  These are HBM/latency-bound integer and byte
// kernels: 16-byte coalesced accesses, LDS counters, wave-level ballots and
// shuffles -- no matrix cores.
//
// The reference contains none of these operations (no router, histogram,
// permutation or combine exists under /root/reference); their semantics are
// the path's frozen specification, restated on the CPU in oracle/spec.py.
#pragma once

#include "common.hpp"

namespace hkmoe {

constexpr int kRouteTok = 32;      // tokens per routing/scatter workgroup
constexpr int kRouteThreads = 256; // scatter: 4 waves per 32-token block
constexpr int kTopkThreads = 512;  // top-k: 8 waves, 4 tokens each (16 lanes per token)
constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 32;
constexpr int kScanThreads = 1024;
constexpr int kTileCounters = 16;  // HKMOE_TILE_COUNTERS
constexpr int kNarrowCounters = 4;  // narrow kernel item counters (GEMM 1, GEMM 2), then their
                                    // active-slot counters

__device__ __forceinline__ bool route_better(float av, int ai, float bv, int bi) {
  if (bi < 0) return ai >= 0;
  if (ai < 0) return false;
  return av > bv || (av == bv && ai < bi);
}

// One level of a row argmax: every lane takes the better of its own entry and
// the one that DPP control CTRL (a permutation within rows of 16 lanes) brings.
template <int CTRL>
__device__ __forceinline__ void route_best_dpp(float& bv, int& bi) {
  const float ov =
      __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(bv), __float_as_int(bv), CTRL, 0xf, 0xf, false));
  const int oi = __builtin_amdgcn_update_dpp(bi, bi, CTRL, 0xf, 0xf, false);
  if (route_better(ov, oi, bv, bi)) {
    bv = ov;
    bi = oi;
  }
}

// ---------------------------------------------------------------------------
// 1. top-k + softmax + per-block histogram.  16 lanes (one row of the wave) per
//    token, 4 tokens per wave; lane s of a token's row holds experts c*16 + s,
//    c < CH (CH: power of two >= ceil(E / 16)).  Each of the k rounds takes
//    the lane's best untaken expert and reduces the row by DPP swaps (quad
//    pairs, quad swap, half-row and row mirrors): VALU only, and a round's
//    work is shared by four tokens.  route_better is a total order, so the
//    reduction order does not change the winner.
// ---------------------------------------------------------------------------
template <int CH>
__global__ __launch_bounds__(kTopkThreads) void route_topk_kernel(
    const float* __restrict__ logits, int num_tokens, int num_experts, int top_k,
    int32_t* __restrict__ topk_idx, float* __restrict__ topk_w, int32_t* __restrict__ block_counts) {
  static_assert(kTopkThreads == 16 * kRouteTok, "one 16-lane row per token");
  static_assert(CH <= 64, "taken mask");
  __shared__ int hist[kMaxExperts];
  const int sub = threadIdx.x & 15;
  for (int e = threadIdx.x; e < num_experts; e += kTopkThreads) hist[e] = 0;
  __syncthreads();

  const int t = blockIdx.x * kRouteTok + (threadIdx.x >> 4);
  if (t < num_tokens) {  // uniform over the token's row
    const float* row = logits + static_cast<int64_t>(t) * num_experts;
    float v[CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int id = c * 16 + sub;
      v[c] = (id < num_experts) ? row[id] : 0.0f;
    }
    uint64_t taken = 0;
    float v0 = 0.0f, mv0 = 0.0f, mv1 = 0.0f;  // winners j (lane j % 16): j < 16 in mv0, else mv1
    int mi0 = 0, mi1 = 0;
    for (int j = 0; j < top_k; ++j) {
      float bv = 0.0f;
      int bi = -1;
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const int id = c * 16 + sub;
        if (id < num_experts && !((taken >> c) & 1u) && route_better(v[c], id, bv, bi)) {
          bv = v[c];
          bi = id;
        }
      }
      route_best_dpp<0xB1>(bv, bi);   // quad_perm [1,0,3,2]
      route_best_dpp<0x4E>(bv, bi);   // quad_perm [2,3,0,1]
      route_best_dpp<0x141>(bv, bi);  // row_half_mirror
      route_best_dpp<0x140>(bv, bi);  // row_mirror
      if ((bi & 15) == sub) taken |= uint64_t{1} << (bi >> 4);
      if (j == 0) v0 = bv;
      if ((j & 15) == sub) {
        if (j < 16) { mv0 = bv; mi0 = bi; } else { mv1 = bv; mi1 = bi; }
      }
    }
    // softmax over the winners: exp(v_j - v_0) / sum_j exp(v_j - v_0), the sum
    // taken in j order
    const float ex0 = (sub < top_k) ? expf(mv0 - v0) : 0.0f;
    const float ex1 = (sub + 16 < top_k) ? expf(mv1 - v0) : 0.0f;
    float tot = 0.0f;
    for (int j = 0; j < top_k; ++j) tot = tot + __shfl(j < 16 ? ex0 : ex1, j & 15, 16);
    if (sub < top_k) {
      topk_idx[static_cast<int64_t>(t) * top_k + sub] = mi0;
      topk_w[static_cast<int64_t>(t) * top_k + sub] = ex0 / tot;
      atomicAdd(&hist[mi0], 1);
    }
    if (sub + 16 < top_k) {
      topk_idx[static_cast<int64_t>(t) * top_k + sub + 16] = mi1;
      topk_w[static_cast<int64_t>(t) * top_k + sub + 16] = ex1 / tot;
      atomicAdd(&hist[mi1], 1);
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < num_experts; e += kTopkThreads)
    block_counts[static_cast<int64_t>(blockIdx.x) * num_experts + e] = hist[e];
}

// ---------------------------------------------------------------------------
// 2. offsets, in two launches.
//  a. expert_block_scan: per expert, the exclusive prefix of its counts over
//     the routing blocks (block_base) and its total (counts).  kOffExperts
//     experts per workgroup, each over kOffParts ranges of blocks, so the
//     block counts are read by many CUs at once (a single workgroup spent
//     most of its time waiting for them).
//  b. expert_offsets: one workgroup of 1024 threads, thread = expert: scans
//     over experts (offsets, M-tile offsets), the M-tile list, counters.
// With at most kOffFuseBlocks routing blocks (decode-sized batches) the
// expert_offsets thread of each expert also does (a) itself, reading the few
// counts in one pass: one launch instead of two.
// ---------------------------------------------------------------------------
constexpr int kOffExperts = 16;                        // experts per block-scan workgroup
constexpr int kOffParts = kScanThreads / kOffExperts;  // block ranges per expert
constexpr int kOffCache = 32;                          // counts a thread keeps in registers
constexpr int kOffFuseBlocks = 16;                     // routing blocks done by expert_offsets

__global__ __launch_bounds__(kScanThreads) void expert_block_scan_kernel(
    const int32_t* __restrict__ block_counts, int nblk, int num_experts, int32_t* __restrict__ counts,
    int32_t* __restrict__ block_base) {
  __shared__ int part_sum[kOffParts][kOffExperts];
  const int tid = threadIdx.x;
  const int el = tid % kOffExperts, part = tid / kOffExperts;
  const int e = blockIdx.x * kOffExperts + el;
  const int per = (nblk + kOffParts - 1) / kOffParts;
  const int b0 = min(nblk, part * per), b1 = min(nblk, b0 + per);
  const bool act = e < num_experts;
  // up to kOffCache counts are loaded at once and kept for the block_base
  // pass; longer ranges are read twice, 16 loads in flight at a time
  const bool cached = per <= kOffCache;
  int cache[kOffCache];
  int s = 0;
  if (act && cached) {
#pragma unroll
    for (int u = 0; u < kOffCache; ++u)
      cache[u] = (b0 + u < b1) ? block_counts[static_cast<int64_t>(b0 + u) * num_experts + e] : 0;
#pragma unroll
    for (int u = 0; u < kOffCache; ++u) s += cache[u];
  } else if (act) {
    for (int b = b0; b < b1; b += 16) {
      int c[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        c[u] = (b + u < b1) ? block_counts[static_cast<int64_t>(b + u) * num_experts + e] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) s += c[u];
    }
  }
  part_sum[part][el] = s;
  __syncthreads();
  if (!act) return;
  // prefix over the ranges before this one, and the expert's total
  int before = 0, total = 0;
  for (int q = 0; q < kOffParts; ++q) {
    const int v = part_sum[q][el];
    if (q < part) before += v;
    total += v;
  }
  if (part == 0) counts[e] = total;
  int run = before;
  if (cached) {
#pragma unroll
    for (int u = 0; u < kOffCache; ++u) {
      if (b0 + u < b1) block_base[static_cast<int64_t>(b0 + u) * num_experts + e] = run;
      run += cache[u];
    }
  } else {
    for (int b = b0; b < b1; b += 16) {
      int c[16];
#pragma unroll
      for (int u = 0; u < 16; ++u)
        c[u] = (b + u < b1) ? block_counts[static_cast<int64_t>(b + u) * num_experts + e] : 0;
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        if (b + u < b1) block_base[static_cast<int64_t>(b + u) * num_experts + e] = run;
        run += c[u];
      }
    }
  }
}

// Exclusive scans of N values per thread over the workgroup, all in one pass.
template <int N>
__device__ __forceinline__ void block_exclusive_scan_n(int (&v)[N], int (*wave_tot)[N]) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl[N];
#pragma unroll
  for (int i = 0; i < N; ++i) incl[i] = v[i];
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int n = __shfl_up(incl[i], o, 64);
      if (lane >= o) incl[i] += n;
    }
  }
  if (lane == 63) {
#pragma unroll
    for (int i = 0; i < N; ++i) wave_tot[wave][i] = incl[i];
  }
  __syncthreads();
  if (wave == 0) {
    const int nw = blockDim.x >> 6;
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int wv = lane < nw ? wave_tot[lane][i] : 0;
      int wi = wv;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int n = __shfl_up(wi, o, 64);
        if (lane >= o) wi += n;
      }
      if (lane < nw) wave_tot[lane][i] = wi - wv;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = wave_tot[wave][i] + incl[i] - v[i];
}

__global__ __launch_bounds__(kScanThreads) void expert_offsets_kernel(
    int num_experts, int32_t* __restrict__ counts, int32_t* __restrict__ offsets,
    int32_t* __restrict__ mtile_offsets, int32_t* __restrict__ mtile_list, int tile_m,
    float* amax_reset, int32_t* tile_counters, int narrow_max, int32_t* narrow_info,
    const int32_t* __restrict__ block_counts, int fused_nblk, int32_t* __restrict__ block_base) {
  __shared__ int wave_tot[kScanThreads / 64][5];
  __shared__ int n_head, n_tail;
  const int e = threadIdx.x;  // E <= kScanThreads
  int cnt = 0;
  if (fused_nblk >= 0) {
    // fused_nblk (<= kOffFuseBlocks) routing blocks: this expert's prefix over
    // them and its total, as expert_block_scan_kernel computes them (-1: the
    // block scan ran before)
    if (e < num_experts) {
      int c[kOffFuseBlocks];
#pragma unroll
      for (int b = 0; b < kOffFuseBlocks; ++b) c[b] = b < fused_nblk ? block_counts[b * num_experts + e] : 0;
#pragma unroll
      for (int b = 0; b < kOffFuseBlocks; ++b) {
        if (b < fused_nblk) block_base[b * num_experts + e] = cnt;
        cnt += c[b];
      }
      counts[e] = cnt;
    }
  } else if (e < num_experts) {
    cnt = counts[e];
  }
  const int mt = (cnt + tile_m - 1) / tile_m;
  // M-tile list [(expert, first row)]: first the experts with at least one
  // full tile, each with all its tiles (full ones, then its partial one), in
  // expert order; then the single partial tiles of the smaller experts; last,
  // with narrow_max > 0, the experts of 1..narrow_max rows, which the narrow
  // kernel takes (their count goes to narrow_info[0]).  Tiles of nearly equal
  // cost sit together in the grouped GEMMs' schedule, so the workgroups that
  // share a tile block stay in step and reuse its operands in L2, and a large
  // expert's partial tile runs while its weights are still in L2 / MALL
  // instead of streaming them once more.
  const int q_full = cnt / tile_m;
  const int q_part = (cnt % tile_m) ? 1 : 0;
  const int q_head = q_full > 0 ? q_full + q_part : 0;
  const int q_narrow = (q_full == 0 && cnt > 0 && cnt <= narrow_max) ? 1 : 0;
  const int q_tail = (q_full > 0 || q_narrow) ? 0 : q_part;
  // one pass of exclusive scans over the experts: row offsets, M-tile
  // offsets, and the list positions of the three kinds of tiles
  int sc[5] = {cnt, mt, q_head, q_tail, q_narrow};
  block_exclusive_scan_n<5>(sc, wave_tot);
  const int off = sc[0], moff = sc[1], head_base = sc[2], tail_base = sc[3], narrow_base = sc[4];
  if (e < num_experts) {
    offsets[e] = off;
    mtile_offsets[e] = moff;
  }
  if (e == num_experts - 1) {
    offsets[num_experts] = off + cnt;
    mtile_offsets[num_experts] = moff + mt;
    n_head = head_base + q_head;
    n_tail = tail_base + q_tail;
    if (mtile_list != nullptr && narrow_info != nullptr) narrow_info[0] = narrow_base + q_narrow;
  }
  if (mtile_list != nullptr) {
    __syncthreads();
    if (e < num_experts) {
      for (int s = 0; s < q_head; ++s) {
        mtile_list[2 * (head_base + s)] = e;
        mtile_list[2 * (head_base + s) + 1] = off + s * tile_m;
      }
      if (q_tail) {
        mtile_list[2 * (n_head + tail_base)] = e;
        mtile_list[2 * (n_head + tail_base) + 1] = off;
      }
      if (q_narrow) {
        mtile_list[2 * (n_head + n_tail + narrow_base)] = e;
        mtile_list[2 * (n_head + n_tail + narrow_base) + 1] = off;
      }
    }
  }
  const int tid = threadIdx.x;
  if (narrow_info != nullptr && tid >= 1 && tid < 1 + kNarrowCounters) narrow_info[tid] = 0;
  if (tid == 0 && amax_reset != nullptr) *amax_reset = 0.0f;
  if (tile_counters != nullptr && tid < kTileCounters) tile_counters[tid] = 0;
}

// ---------------------------------------------------------------------------
// 3. stable scatter + row gather.  Same token chunks as route_topk_kernel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kRouteThreads) void scatter_kernel(
    const int32_t* __restrict__ topk_idx, int num_tokens, int num_experts, int top_k,
    const int32_t* __restrict__ offsets, const int32_t* __restrict__ block_base,
    int32_t* __restrict__ perm, int32_t* __restrict__ inv_perm, const uint8_t* __restrict__ x_q,
    const float* __restrict__ x_scale, int64_t hidden, int block_scaled, uint8_t* __restrict__ xp,
    float* __restrict__ xps_t, int64_t rows_total) {
  __shared__ int ctr[kMaxExperts];
  __shared__ int pos[kRouteTok * kMaxTopK];
  const int lane = threadIdx.x & 63;
  const int t0 = blockIdx.x * kRouteTok;
  const int ntok = min(kRouteTok, num_tokens - t0);
  const int nslot = ntok * top_k;
  const int64_t f0 = static_cast<int64_t>(t0) * top_k;
  for (int e = threadIdx.x; e < num_experts; e += kRouteThreads)
    ctr[e] = offsets[e] + block_base[static_cast<int64_t>(blockIdx.x) * num_experts + e];
  __syncthreads();

  if (threadIdx.x < 64) {
    int nbits = 0;
    while ((1 << nbits) < num_experts) ++nbits;
    for (int s0 = 0; s0 < nslot; s0 += 64) {
      const int s = s0 + lane;
      const bool valid = s < nslot;
      const int e = valid ? topk_idx[f0 + s] : 0;
      uint64_t peers = __ballot(valid);
      for (int b = 0; b < nbits; ++b) {
        const bool bit = (e >> b) & 1;
        const uint64_t bal = __ballot(bit);
        peers &= bit ? bal : ~bal;
      }
      const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      const int rank = __popcll(peers & lt);
      const int leader = valid ? (__ffsll(static_cast<long long>(peers)) - 1) : 0;
      int base = 0;
      if (valid && lane == leader) base = atomicAdd(&ctr[e], __popcll(peers));
      base = __shfl(base, leader, 64);
      if (valid) {
        const int p = base + rank;
        perm[p] = static_cast<int32_t>(f0 + s);
        inv_perm[f0 + s] = p;
        pos[s] = p;
      }
    }
  }
  __syncthreads();
  if (x_q == nullptr) return;

  // gather: each token row is read once and written to its top_k destinations
  const int64_t chunks = hidden / 16;
  const int64_t work = static_cast<int64_t>(ntok) * chunks;
  for (int64_t w = threadIdx.x; w < work; w += kRouteThreads) {
    const int tt = static_cast<int>(w / chunks);
    const int64_t c = w - static_cast<int64_t>(tt) * chunks;
    const uint4 v = *reinterpret_cast<const uint4*>(x_q + static_cast<int64_t>(t0 + tt) * hidden + c * 16);
    for (int j = 0; j < top_k; ++j) {
      const int p = pos[tt * top_k + j];
      *reinterpret_cast<uint4*>(xp + static_cast<int64_t>(p) * hidden + c * 16) = v;
    }
  }
  if (block_scaled) {
    const int groups = static_cast<int>(hidden / kGroup);
    const int swork = ntok * groups;
    for (int w = threadIdx.x; w < swork; w += kRouteThreads) {
      const int tt = w / groups, g = w - tt * groups;
      const float sv = x_scale[static_cast<int64_t>(t0 + tt) * groups + g];
      for (int j = 0; j < top_k; ++j)
        xps_t[static_cast<int64_t>(g) * rows_total + pos[tt * top_k + j]] = sv;
    }
  }
}

// ---------------------------------------------------------------------------
// 4. requantisation of the bf16 intermediate
// ---------------------------------------------------------------------------
// 1x128 groups: one workgroup (256 threads) per row, one wave per group.
__global__ __launch_bounds__(256) void requant_group_kernel(const uint16_t* __restrict__ h,
                                                            int64_t rows, int inter,
                                                            uint8_t* __restrict__ hq,
                                                            float* __restrict__ hs_t) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t r = blockIdx.x;
  const int groups = inter / kGroup;
  for (int g = wave; g < groups; g += 4) {
    const int64_t base = r * inter + g * kGroup + lane * 2;
    const uint32_t pair = *reinterpret_cast<const uint32_t*>(h + base);
    const float a = bf16_bits_to_f32(pair & 0xffffu), b = bf16_bits_to_f32(pair >> 16);
    const float amax = wave_max(fmaxf(fabsf(a), fabsf(b)));
    const float s = scale_from_amax(amax);
    const uint32_t q = pack_e4m3x4(quot_e4m3(a, s), quot_e4m3(b, s), 0.0f, 0.0f) & 0xffffu;
    *reinterpret_cast<uint16_t*>(hq + base) = static_cast<uint16_t>(q);
    if (lane == 0) hs_t[static_cast<int64_t>(g) * rows + r] = s;
  }
}

// per-tensor: amax was accumulated by GEMM 1 over the bf16-rounded h, so s is
// the scale of a bf16 maximum and every x is a bf16 value: the division-free
// quotient (QuotScale) gives the bytes of x / s there, as the GEMM epilogues'
// self-check establishes for that domain.  One case lies outside it: an
// infinite x with a finite s (amax NaN, s = 1), where x / s is x (saturated by
// the conversion) and the remainder step would give NaN.  8 elements per
// 16-byte chunk; each thread issues its 4 chunks' loads (read once:
// non-temporal) before converting any, so 4 KiB per wave are in flight.
__global__ __launch_bounds__(256) void requant_tensor_kernel(const uint16_t* __restrict__ h,
                                                             int64_t n8, const float* amax,
                                                             uint8_t* __restrict__ hq,
                                                             float* __restrict__ hs) {
  constexpr int kU = 4;
  const float s = scale_from_amax(*amax);
  const QuotScale qs = quot_scale(s);
  const bool s_finite = !__builtin_isinf(s);
  if (blockIdx.x == 0 && threadIdx.x == 0) hs[0] = s;
  auto quot = [&](uint32_t bits) __attribute__((always_inline)) {
    const float x = bf16_bits_to_f32(bits);
    const float q = quot_e4m3(x, qs);
    return (s_finite && __builtin_isinf(x)) ? x : q;
  };
  auto convert = [&](uint4 v) __attribute__((always_inline)) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint2 o;
    uint32_t* op = &o.x;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const uint32_t p0 = w[q * 2], p1 = w[q * 2 + 1];
      op[q] = pack_e4m3x4(quot(p0 & 0xffffu), quot(p0 >> 16), quot(p1 & 0xffffu), quot(p1 >> 16));
    }
    return o;
  };
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  int64_t i = blockIdx.x * 256ll + threadIdx.x;
  for (; i + (kU - 1) * stride < n8; i += kU * stride) {
    uint4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) v[u] = ld_nt16(h + (i + u * stride) * 8);
#pragma unroll
    for (int u = 0; u < kU; ++u) reinterpret_cast<uint2*>(hq)[i + u * stride] = convert(v[u]);
  }
  for (; i < n8; i += stride) reinterpret_cast<uint2*>(hq)[i] = convert(ld_nt16(h + i * 8));
}

// ---------------------------------------------------------------------------
// 5. combine: out[t] = bf16(sum_j w[t,j] * y[inv_perm[t*k+j]]), one
//    workgroup per token, 8 columns (16 bytes) per thread and step (the
//    host sizes the workgroup so the row's 16-byte chunks divide evenly).  The
//    token's weights and y rows are staged in LDS once; the y loads of up to
//    8 slots are issued together, then summed in slot order j = 0 .. k-1.
//    Every y byte is read once and every out byte written once: non-temporal
//    loads and stores (181 vs 208 us on config 3).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(512) void combine_kernel(const uint16_t* __restrict__ y,
                                                      const float* __restrict__ topk_w,
                                                      const int32_t* __restrict__ inv_perm,
                                                      int top_k, int hidden,
                                                      uint16_t* __restrict__ out) {
  __shared__ float s_w[kMaxTopK];
  __shared__ int32_t s_row[kMaxTopK];
  const int64_t t = blockIdx.x;
  if (threadIdx.x < top_k) {
    s_w[threadIdx.x] = topk_w[t * top_k + threadIdx.x];
    s_row[threadIdx.x] = inv_perm[t * top_k + threadIdx.x];
  }
  __syncthreads();
  const int cols8 = hidden / 8;
  for (int c = threadIdx.x; c < cols8; c += blockDim.x) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < top_k; j0 += 8) {
      uint4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (j0 + u < top_k)
          v[u] = ld_nt16(y + static_cast<int64_t>(s_row[j0 + u]) * hidden + c * 8);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (j0 + u < top_k) {
          const float w = s_w[j0 + u];
          const uint32_t wv[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[2 * q] = acc[2 * q] + w * bf16_bits_to_f32(wv[q] & 0xffffu);
            acc[2 * q + 1] = acc[2 * q + 1] + w * bf16_bits_to_f32(wv[q] >> 16);
          }
        }
      }
    }
    uint4 o;
    o.x = pack_bf16x2(acc[0], acc[1]);
    o.y = pack_bf16x2(acc[2], acc[3]);
    o.z = pack_bf16x2(acc[4], acc[5]);
    o.w = pack_bf16x2(acc[6], acc[7]);
    st_nt16(out + t * hidden + c * 8, o);
  }
}

// ---------------------------------------------------------------------------
// Self-check of the epilogues' requantisation quotient: quot_e4m3(x, qs)
// against the correctly rounded x / s for every input the GEMM epilogues can
// produce: x a bf16 value, s = scale_from_amax(amax) with amax a bf16 value
// >= |x|.  Both quotients scale exactly with powers of two, so the check
// enumerates mantissas and sampled exponents: blocks (ma, ea) with amax =
// (1 + ma/128) 2^ea, ea = -126, -119, ..., 126; threads mx; each thread tries
// x = +-(1 + mx/128) 2^(ea - g), g = 0 .. 40 (x <= amax, x normal), and, in
// blocks with y in 37 .. 63, bf16 subnormals and zeros x = +-mx 2^-133
// against amax with ea in [-126, -100]; blocks with y = 64, amax = +inf (a row
// whose h overflowed) against finite and infinite x.  counts[0] += cases,
// counts[1] += mismatches: e4m3 bytes that differ, or fp32 quotients that
// differ where |x / s| >= 2^-10 (signed zeros included; two NaNs agree).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(128) void requant_quotient_check_kernel(int* __restrict__ counts) {
  const int ma = blockIdx.x, mx = threadIdx.x;
  if (blockIdx.y == 64) {
    // a row whose h overflowed: amax = +inf, s = +inf; x = +-(1 + mx/128) 2^e for
    // e = -126 + ma*2 (block ma < 127), or x = +-inf (block 127, thread 0)
    const QuotScale qs = quot_scale(scale_from_amax(__builtin_inff()));
    const float s = scale_from_amax(__builtin_inff());
    int cases = 0, bad = 0;
    if (ma < 127 || mx == 0) {
      const float x = ma < 127 ? __builtin_amdgcn_ldexpf(1.0f + mx / 128.0f, -126 + 2 * ma) : __builtin_inff();
#pragma unroll
      for (int sg = 0; sg < 2; ++sg) {
        const float xv = sg ? -x : x;
        const float qd = quot_e4m3(xv, s), qm = quot_e4m3(xv, qs);
        // both NaN (inf / inf; its sign is not specified), or the same bits
        bad += !((__builtin_isnan(qd) && __builtin_isnan(qm)) || __float_as_uint(qd) == __float_as_uint(qm));
        ++cases;
      }
    }
    atomicAdd(&counts[0], cases);
    atomicAdd(&counts[1], bad);
    return;
  }
  const bool sub = blockIdx.y >= 37;
  const int ea = sub ? -126 + static_cast<int>(blockIdx.y - 37) : -126 + 7 * static_cast<int>(blockIdx.y);
  const float amax = __builtin_amdgcn_ldexpf(1.0f + ma / 128.0f, ea);
  const float s = scale_from_amax(amax);
  const QuotScale qs = quot_scale(s);
  int cases = 0, bad = 0;
  for (int g = 0; g <= (sub ? 0 : 40); ++g) {
    float x;
    if (sub) {
      x = __builtin_amdgcn_ldexpf(static_cast<float>(mx), -133);  // mx = 0: +-0
    } else {
      if (ea - g < -126) break;
      if (g == 0 && mx > ma) continue;  // x <= amax
      x = __builtin_amdgcn_ldexpf(1.0f + mx / 128.0f, ea - g);
    }
#pragma unroll
    for (int sg = 0; sg < 2; ++sg) {
      const float xv = sg ? -x : x;
      const float qd = quot_e4m3(xv, s), qm = quot_e4m3(xv, qs);
      // the stored e4m3 bytes must agree, and the fp32 quotients too wherever
      // they can round to a nonzero e4m3 value
      const bool same_byte = (pack_e4m3x4(qd, 0.0f, 0.0f, 0.0f) & 0xffu) == (pack_e4m3x4(qm, 0.0f, 0.0f, 0.0f) & 0xffu);
      const bool same_bits = __float_as_uint(qd) == __float_as_uint(qm) || fabsf(qd) < 0.0009765625f;
      bad += !(same_byte && same_bits);
      ++cases;
    }
  }
  atomicAdd(&counts[0], cases);
  atomicAdd(&counts[1], bad);
}

// ---------------------------------------------------------------------------
// 6. quantisers (fp32 input) used to build e4m3 operands on the device
// ---------------------------------------------------------------------------
// 1x128 groups, row-major scales [R, C/128]; one wave per group.
__global__ __launch_bounds__(256) void quant_group_kernel(const float* __restrict__ x, int64_t rows,
                                                          int64_t cols, uint8_t* __restrict__ q,
                                                          float* __restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int64_t gid = blockIdx.x * 4ll + (threadIdx.x >> 6);
  const int64_t groups = cols / kGroup;
  if (gid >= rows * groups) return;
  const int64_t r = gid / groups, g = gid - r * groups;
  const int64_t base = r * cols + g * kGroup + lane * 2;
  const float2 v = *reinterpret_cast<const float2*>(x + base);
  const float amax = wave_max(fmaxf(fabsf(v.x), fabsf(v.y)));
  const float sc = scale_from_amax(amax);
  const uint32_t qq = f32_to_e4m3(v.x / sc) | (f32_to_e4m3(v.y / sc) << 8);
  *reinterpret_cast<uint16_t*>(q + base) = static_cast<uint16_t>(qq);
  if (lane == 0) s[gid] = sc;
}

// 128x128 blocks of [B, R, C]; one workgroup (256 threads) per block.
__global__ __launch_bounds__(256) void quant_block_kernel(const float* __restrict__ x, int64_t rows,
                                                          int64_t cols, uint8_t* __restrict__ q,
                                                          float* __restrict__ s) {
  __shared__ float red[4];
  const int64_t bc = cols / kGroup, br = rows / kGroup;
  const int64_t blk = blockIdx.x;
  const int64_t b = blk / (br * bc);
  const int64_t rem = blk - b * br * bc;
  const int64_t bi = rem / bc, bj = rem - bi * bc;
  const float* xb = x + (b * rows + bi * kGroup) * cols + bj * kGroup;
  uint8_t* qb = q + (b * rows + bi * kGroup) * cols + bj * kGroup;
  // thread: rows (tid/32) + 8*u, columns 4*(tid%32) .. +3
  const int cr = threadIdx.x >> 5, cc = (threadIdx.x & 31) * 4;
  float m = 0.0f;
  for (int u = 0; u < 16; ++u) {
    const float4 v = *reinterpret_cast<const float4*>(xb + static_cast<int64_t>(cr + 8 * u) * cols + cc);
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  const float amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float sc = scale_from_amax(amax);
  for (int u = 0; u < 16; ++u) {
    const int64_t off = static_cast<int64_t>(cr + 8 * u) * cols + cc;
    const float4 v = *reinterpret_cast<const float4*>(xb + off);
    const uint32_t qq = f32_to_e4m3(v.x / sc) | (f32_to_e4m3(v.y / sc) << 8) |
                        (f32_to_e4m3(v.z / sc) << 16) | (f32_to_e4m3(v.w / sc) << 24);
    *reinterpret_cast<uint32_t*>(qb + off) = qq;
  }
  if (threadIdx.x == 0) s[blk] = sc;
}

__global__ __launch_bounds__(256) void amax_kernel(const float* __restrict__ x, int64_t n,
                                                   float* amax) {
  float m = 0.0f;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    m = fmaxf(m, fabsf(x[i]));
  m = wave_max(m);
  if ((threadIdx.x & 63) == 0) atomicMax(reinterpret_cast<unsigned int*>(amax), __float_as_uint(m));
}

__global__ void fill_f32_kernel(float* p, float v) { *p = v; }

__global__ __launch_bounds__(256) void quant_tensor_kernel(const float* __restrict__ x, int64_t n,
                                                           const float* amax,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ s) {
  const float sc = scale_from_amax(*amax);
  if (blockIdx.x == 0 && threadIdx.x == 0) s[0] = sc;
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    q[i] = static_cast<uint8_t>(f32_to_e4m3(x[i] / sc));
}

// ---------------------------------------------------------------------------
// 7. MX (e8m0 1x32) operands
// ---------------------------------------------------------------------------
// x viewed as [blocks, 32] (row-major [R, C] with C % 32 == 0): 8 lanes per
// block, 4 elements each.  s = biased exponent of amax = clamp(floor(log2 amax)
// + 127, 0, 254) -- exact for every finite amax (0 for zero or subnormal amax)
// -- and q = e4m3(x * 2^(127 - s)), an exact power-of-two scaling followed by
// one RNE conversion (|x * 2^(127-s)| < 2, so the saturating clamp never acts).
// Reference behaviour: 4_wave.cu:296-321, 368-373.
__global__ __launch_bounds__(256) void quant_mx_kernel(const float* __restrict__ x, int64_t blocks,
                                                       uint8_t* __restrict__ q, uint8_t* __restrict__ s) {
  const int64_t quads = blocks * 8;
  // quad i = lane i % 8 of block i / 8; the 8 lanes of a block sit in one wave
  // (i % 8 == threadIdx.x % 8) and pass the loop test together
  for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < quads; i += static_cast<int64_t>(gridDim.x) * 256) {
    const float4 v = *reinterpret_cast<const float4*>(x + 4 * i);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    m = fmaxf(m, __shfl_xor(m, 1, kWave));
    m = fmaxf(m, __shfl_xor(m, 2, kWave));
    m = fmaxf(m, __shfl_xor(m, 4, kWave));
    const uint32_t e = min((__float_as_uint(m) >> 23) & 0xffu, 254u);
    const int sh = 127 - static_cast<int>(e);
    *reinterpret_cast<uint32_t*>(q + 4 * i) =
        pack_e4m3x4(__builtin_amdgcn_ldexpf(v.x, sh), __builtin_amdgcn_ldexpf(v.y, sh),
                    __builtin_amdgcn_ldexpf(v.z, sh), __builtin_amdgcn_ldexpf(v.w, sh));
    if ((i & 7) == 0) s[i >> 3] = static_cast<uint8_t>(e);
  }
}

// e8m0 s [R, C/32] -> packed words [C/128, R64] (R64 = R rounded up to 64):
// word (kt, p) byte g = s[64*(p/64) + 16*g + p%16][4*kt + (p%64)/16], 0 past
// row R.  One thread per word.  Same words as the reference's pack_scales_kernel
// + repack_scales_for_mfma_kernel (4_wave.cu:323-364) when R % 64 == 0.
__global__ __launch_bounds__(256) void mx_pack_scales_kernel(const uint8_t* __restrict__ s, int64_t rows,
                                                             int64_t kblocks, int64_t rows64,
                                                             uint32_t* __restrict__ packed,
                                                             int64_t words) {
  for (int64_t w = blockIdx.x * 256ll + threadIdx.x; w < words; w += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t kt = w / rows64, p = w - kt * rows64;
    const int64_t r0 = (p & ~63ll) + (p & 15);
    const int64_t kb = 4 * kt + ((p >> 4) & 3);
    uint32_t v = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t r = r0 + 16 * g;
      if (r < rows) v |= static_cast<uint32_t>(s[r * kblocks + kb]) << (8 * g);
    }
    packed[w] = v;
  }
}

// Weight exponents e8m0 [E, nb, K/32] -> the grouped MX GEMM's words, per B
// tile: [E][nb/256][K/128][256], word p of (expert e, N tile nt, K step kt)
// holds in byte g the exponent of B-tile row R = 64*(p/64) + 16g + p%16 for K
// block 4kt + (p%64)/16.  B-tile row R is weight row nt*256 + R, or for the
// fused gate/up weights (gate_up = I) row nt*128 + 32*(R>>6) + (R&31) +
// ((R>>5)&1)*I: the row order of pack_weights_kernel's stage images.
__global__ __launch_bounds__(256) void mx_pack_weight_words_kernel(const uint8_t* __restrict__ s, int64_t nb,
                                                                   int K, int gate_up,
                                                                   uint32_t* __restrict__ out,
                                                                   int64_t words) {
  const int ks = K / 128, kb = K / 32;
  const int64_t ntile = nb / 256;
  for (int64_t w = blockIdx.x * 256ll + threadIdx.x; w < words; w += static_cast<int64_t>(gridDim.x) * 256) {
    const int pos = static_cast<int>(w & 255);
    const int64_t t = w >> 8;
    const int kt = static_cast<int>(t % ks);
    const int64_t tile = t / ks;
    const int64_t e = tile / ntile;
    const int nt = static_cast<int>(tile - e * ntile);
    const int blk = 4 * kt + ((pos >> 4) & 3);
    uint32_t v = 0;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int R = (pos & ~63) + 16 * g + (pos & 15);
      const int64_t wrow = gate_up ? nt * 128 + 32 * (R >> 6) + (R & 31) + ((R >> 5) & 1) * gate_up
                                   : static_cast<int64_t>(nt) * 256 + R;
      v |= static_cast<uint32_t>(s[(e * nb + wrow) * kb + blk]) << (8 * g);
    }
    out[w] = v;
  }
}

// Activation exponents e8m0 [x_rows, K/32] -> tile-aligned words in expert
// order: [K/128][ws_rs], word m*256 + q of K step kt (M tile m in expert order,
// first row row0, `valid` rows) holds in byte g the exponent of tile row
// r = 64*(q/64) + 16g + q%16 -- output row row0 + r, read from x row
// gather[row0 + r] / gather_div (or row0 + r) -- for K block 4kt + (q%64)/16;
// 0 for r >= valid.
// One workgroup per M tile: the tile's expert is found once, its (gathered)
// rows' exponent bytes are copied into LDS as whole rows (4-byte loads along
// each row), and thread q then writes word q of every K step (consecutive
// threads, consecutive words).  K <= 16384: at most 512 bytes per row.
constexpr int kMxGatherMaxKb = 16384 / 32;
__global__ __launch_bounds__(256) void mx_gather_words_kernel(const uint8_t* __restrict__ s, int K,
                                                              const int32_t* __restrict__ gather, int gather_div,
                                                              const int32_t* __restrict__ offsets,
                                                              const int32_t* __restrict__ mtile_offsets,
                                                              int num_experts, int64_t ws_rs,
                                                              uint32_t* __restrict__ out) {
  extern __shared__ __attribute__((aligned(16))) uint8_t rows_s[];  // [256][kb] exponent bytes
  __shared__ int s_row0, s_valid;
  __shared__ int64_t xrow_s[256];  // x row of each tile row, -1 past `valid`
  const int kb = K / 32, ks = K / 128;
  const int n_mt = mtile_offsets[num_experts];
  const int tid = threadIdx.x;
  for (int m = blockIdx.x; m < n_mt; m += gridDim.x) {
    if (tid == 0) {
      int lo = 0, hi = num_experts;  // largest e with mtile_offsets[e] <= m
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (mtile_offsets[mid] <= m) lo = mid; else hi = mid;
      }
      const int row0 = offsets[lo] + (m - mtile_offsets[lo]) * 256;
      s_row0 = row0;
      s_valid = min(256, offsets[lo + 1] - row0);
    }
    __syncthreads();
    {
      const int row0 = s_row0, valid = s_valid;
      xrow_s[tid] = tid < valid ? (gather ? gather[row0 + tid] / gather_div : row0 + tid) : -1;
    }
    __syncthreads();
    // the rows' bytes in chunks of 16 (K a multiple of 512 and s 16-byte
    // aligned) or 4, up to 16 loads in flight per thread; rows past `valid`
    // read as zero bytes
    auto copy_rows = [&](auto chunk_tag) __attribute__((always_inline)) {
      using C = decltype(chunk_tag);
      constexpr int kC = sizeof(C);
      const int per_row = kb / kC, total = 256 * per_row;
      for (int base = 0; base < total; base += 256 * 16) {
        C v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int i = base + u * 256 + tid;
          v[u] = C{};
          if (i < total) {
            const int r = i / per_row, c = i - r * per_row;
            const int64_t xr = xrow_s[r];
            if (xr >= 0) v[u] = reinterpret_cast<const C*>(s + xr * kb)[c];
          }
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int i = base + u * 256 + tid;
          if (i < total) reinterpret_cast<C*>(rows_s)[i] = v[u];
        }
      }
    };
    if (kb % 16 == 0 && (reinterpret_cast<uintptr_t>(s) & 15) == 0) copy_rows(uint4{}); else copy_rows(uint32_t{});
    __syncthreads();
    const int q = tid;
    const int rbase = (q & ~63) + (q & 15), bsub = (q >> 4) & 3;
    uint32_t* dst = out + static_cast<int64_t>(m) * 256 + q;
    for (int kt = 0; kt < ks; ++kt) {
      const int blk = 4 * kt + bsub;
      uint32_t v = 0;
#pragma unroll
      for (int g = 0; g < 4; ++g) v |= static_cast<uint32_t>(rows_s[(rbase + 16 * g) * kb + blk]) << (8 * g);
      dst[static_cast<int64_t>(kt) * ws_rs] = v;
    }
    __syncthreads();  // rows_s is rewritten for the next M tile
  }
}

}  // namespace hkmoe
