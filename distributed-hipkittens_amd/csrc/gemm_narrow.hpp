// Narrow grouped GEMM for small expert segments (at most 64 rows), block
// scales, gfx950.
//
// A segment of <= 64 rows against a 256-row weight panel does 2*64*256*K
// FLOPs for 256*K weight bytes: it is bound by streaming the weights from HBM,
// not by the MFMA.  The 256x256 persistent kernel (gemm_fp8.hpp) keeps only
// two K steps of weights in flight per CU and needs the whole CU's LDS for
// them, so such tiles run at HBM latency.  This kernel streams the weights
// straight into VGPRs instead, P K steps ahead (P * 4 KiB per wave, 256 KiB
// per CU at P = 8), so a few dozen CUs can pull HBM bandwidth while the other
// CUs run the compute-bound 256x256 tiles of the large experts (the host
// launches the two kernels on two streams).
//
//  * work item: (narrow segment m, 256-row N tile nt), taken from one atomic
//    counter; while the list also holds 256x256 tiles only narrow_active
//    workgroups take items, the first ones to start (a second counter), and
//    the others exit at once and leave their CUs to the 256x256 kernel; else
//    every workgroup of the launch (one per CU) does.  Segment m is
//    entry first + m of the M-tile list (the narrow experts are listed last).
//  * 8 waves; wave w owns 32 weight rows = two 16-row fragments:
//      gate/up GEMM: gate rows 16w..16w+15 of the tile's 128 and the matching
//                    up rows (h columns 16w..16w+15);
//      plain GEMM:   rows 32w..32w+31 of the 256.
//    Each lane loads its fragment rows' 32 K bytes per step with two 16-byte
//    buffer loads per fragment, in the register order read_frag produces from
//    LDS: the MFMA operands, the block-scale arithmetic and the epilogue are those
//    of the 256x256 kernel, so both kernels give the same bits.
//  * activations: every wave DMAs 8 of the segment's 64 rows (rows past the
//    segment repeat its last row) into an LDS ring of P+1 stages, loaded P
//    steps ahead like the weights; one barrier per K step.  An item's
//    activation and weight scales for all its K steps are DMA'd into one of two
//    LDS buffers once, when the item is decoded (at least P steps before its
//    first step).
//  * every wave issues exactly 5 vector-memory instructions per K step (A rows,
//    4 weight loads), so "step kt has landed" is vmcnt(5*(P-1)) (other loads
//    only add to the count, so the wait can only be longer); after the last
//    item the loads continue on that item's first steps (valid addresses, never
//    read), so the count never changes.
//  * K steps per item must be a multiple of P, so a group of P unrolled steps
//    never straddles two items; the loads of an item's last group are the next
//    item's first P steps.
//  * the compiler must not wait for the prefetch window by itself: LDS
//    accesses and the item decode's scalar loads are inline asm with their own
//    lgkmcnt waits (it would otherwise wait for every buffer->LDS DMA before an
//    LDS access, and for pending stores before a scalar load), and the next
//    item's gathered row indices reach LDS by a DMA issued a group before they
//    are read.
#pragma once

#include "gemm_fp8.hpp"

namespace hkmoe {

constexpr int kNarrowRows = 64;
constexpr int kNarrowAStage = kNarrowRows * kBK;                  // 8 KiB of A rows
constexpr int kNarrowStage = kNarrowAStage;                       // one ring stage: A rows
constexpr int kNarrowMaxSteps = 64;                               // K <= 8192
// per-item scales, two buffers (current / next item): [K step][64 rows] activation
// scales, then per wave [2 block rows][K step] weight scales
constexpr int kNarrowWsOff = kNarrowMaxSteps * kNarrowRows * 4;  // 16 KiB
constexpr int kNarrowScaleBuf = kNarrowWsOff + 8 * 2 * kNarrowMaxSteps * 4;
constexpr int kNarrowCtLd = 128 + 8;                              // staged h row (bf16)
constexpr int kNarrowVmPerStep = 5;

constexpr int narrow_ct_off(int P) { return (P + 1) * kNarrowStage; }
constexpr int narrow_gidx_off(int P) { return narrow_ct_off(P) + kNarrowRows * kNarrowCtLd * 2; }
constexpr int narrow_q_off(int P) { return narrow_gidx_off(P) + 8 * 256; }
constexpr int narrow_scale_off(int P) { return narrow_q_off(P) + 256; }
constexpr int narrow_lds_bytes(int P) {
  // ring, h staging tile, per-wave gathered row indices, published item index, scales
  return narrow_scale_off(P) + 2 * kNarrowScaleBuf;
}
static_assert(narrow_lds_bytes(8) <= 160 * 1024, "LDS budget");

extern "C" __device__ i32x4 hk_raw_buffer_load_v4i32(i32x4 rsrc, int voffset, int soffset,
                                                     int aux) __asm("llvm.amdgcn.raw.buffer.load.v4i32");

// a[idx] for a wave-uniform idx through the scalar cache, complete on return.
// Only for data written before the kernel started.
__device__ __forceinline__ int sload_i32(const int32_t* a, int idx) {
  const i32x4 srd = make_srd(a, 0xffffffffu);
  const int off = __builtin_amdgcn_readfirstlane(idx * 4);
  int v;
  asm volatile("s_buffer_load_dword %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=&s"(v) : "s"(srd), "s"(off));
  return v;
}

template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// LDS accesses of the narrow kernel are written as inline asm with their own
// lgkmcnt waits; outputs are early-clobber ("=&"), since a load's destination
// is written after later instructions of the same block have read their
// address registers.  The compiler cannot tell the ring slots apart, so before any
// LDS access it can see it would wait for every buffer->LDS DMA still in
// flight, i.e. for the whole prefetch window.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// One A fragment (two 16-byte chunks at a_lo / a_hi + OFF) and its row scale
// (a_sc + SOFF), complete on return.
template <int OFF, int SOFF>
__device__ __forceinline__ void lds_frag(uint32_t a_lo, uint32_t a_hi, uint32_t a_sc, i32x8& f, float& sc) {
  i32x4 lo, hi;
  asm volatile(
      "ds_read_b128 %0, %3 offset:%6\n\t"
      "ds_read_b128 %1, %4 offset:%6\n\t"
      "ds_read_b32 %2, %5 offset:%7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(lo), "=&v"(hi), "=&v"(sc)
      : "v"(a_lo), "v"(a_hi), "v"(a_sc), "i"(OFF), "i"(SOFF));
  f.lo = lo;
  f.hi = hi;
}

__device__ __forceinline__ float2 lds_read_f2(uint32_t a) {
  float2 v;
  asm volatile("ds_read_b64 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
  return v;
}

// the dwords at a and a + 256 (an item's two weight-scale rows at one K step)
__device__ __forceinline__ float2 lds_read_w2(uint32_t a) {
  float x, y;
  asm volatile("ds_read_b32 %0, %2\n\tds_read_b32 %1, %2 offset:256\n\ts_waitcnt lgkmcnt(0)"
               : "=&v"(x), "=&v"(y)
               : "v"(a));
  return float2{x, y};
}

__device__ __forceinline__ int lds_read_i32(uint32_t a) {
  int v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
  return v;
}

__device__ __forceinline__ void lds_write_i32(uint32_t a, int v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}

__device__ __forceinline__ void lds_write_b64(uint32_t a, uint2 v) {
  asm volatile("ds_write_b64 %0, %1" ::"v"(a), "v"(v) : "memory");
}

// 16 bytes at a, complete on return
__device__ __forceinline__ uint4 lds_read_u4(uint32_t a) {
  uint4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(v) : "v"(a));
  return v;
}

// LDS writes done, then the workgroup barrier (no vmcnt: DMA stays in flight)
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <Epi EPI, int P>
__global__ __launch_bounds__(kThreads, 1) void gemm_fp8_narrow(GemmParams p) {
  static_assert(EPI == Epi::kSiluQuant || EPI == Epi::kStoreBf16, "narrow epilogues");
  static_assert(P == 2 || P == 4 || P == 8, "prefetch depth");
  static_assert(kNarrowVmPerStep * (P - 1) <= 63, "vmcnt range");
  constexpr bool kSilu = (EPI == Epi::kSiluQuant);
  constexpr int kRing = P + 1;
  extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
  uint16_t* ct = reinterpret_cast<uint16_t*>(smem + narrow_ct_off(P));
  int32_t* gidx = reinterpret_cast<int32_t*>(smem + narrow_gidx_off(P));

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int lg = lane >> 4;
  const int fx = swz(l16);

  const int k_steps = p.K / kBK;
  const int groups = k_steps / P;
  const int total_mt = sload_i32(p.mtile_offsets, p.num_experts);
  const int n_narrow = sload_i32(p.narrow_cnt, 0);
  const int first = total_mt - n_narrow;
  const int n_items = n_narrow * p.n_tiles;
  // beside 256x256 tiles only narrow_active workgroups take items (the others
  // exit and leave their CUs to the 256x256 kernel); alone, all of them do
  if (n_items <= 0) return;
  int32_t* const item_ctr = p.tile_ctr;  // zeroed item counter; p.tile_ctr[2]: active slots
  int* s_q = reinterpret_cast<int*>(smem + narrow_q_off(P));  // published item index

  // this wave's two fragment rows, tile-local (row R of the 256-row tile;
  // fragment R/16 of the packed block) and relative to the N tile's first
  // weight row
  int frag_r[2], frag_w[2];
  if constexpr (kSilu) {
    frag_r[0] = 64 * (wave >> 1) + 16 * (wave & 1) + l16;  // gate row 16w + l16 of the tile
    frag_r[1] = frag_r[0] + 32;                             // its up row
    frag_w[0] = 16 * wave + l16;                            // + nt*128
    frag_w[1] = 16 * wave + l16 + p.n_out;                  // + nt*128 (up half starts at I)
  } else {
    frag_r[0] = 32 * wave + l16;
    frag_r[1] = 32 * wave + 16 + l16;
    frag_w[0] = frag_r[0];                                  // + nt*256
    frag_w[1] = frag_r[1];
  }
  const int ld_row = 8 * wave + (lane >> 3);                // A row this lane DMAs
  const int ld_chunk = (lane & 7) ^ swz(ld_row);
  const i32x4 a_srd = make_srd(p.a, p.a_bytes);
  const i32x4 as_srd = make_srd(p.a_scale, 0xffffffffu);
  const i32x4 g_srd = make_srd(p.a_gather, 0xffffffffu);
  const int64_t kb_per_expert = static_cast<int64_t>(p.nb / kGroup) * k_steps;

  // Lane-constant weight offsets within a K step: packed layout, the two
  // contiguous 1 KiB register halves of the fragment (one load each, whole
  // 128-byte lines); row-major, the weight row (relative to the item's first
  // row, which goes into the descriptor).
  int wvoff[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    if (p.b_packed) {
      // fragment-major block: fragment f's register halves are 1 KiB each
      const int f = frag_r[j] >> 4;
      wvoff[2 * j] = (2 * f) * 1024 + lane * 16;
      wvoff[2 * j + 1] = (2 * f + 1) * 1024 + lane * 16;
    } else {
      wvoff[2 * j] = buf_off(frag_w[j], p.K, (2 * lg) * 16);
      wvoff[2 * j + 1] = buf_off(frag_w[j], p.K, (2 * lg + 1) * 16);
    }
  }
  // lane-constant LDS offsets within a ring stage: A fragment chunks of row
  // l16 (fragment i adds 2 KiB), its row scale (fragment i adds 64 bytes), and
  // this wave's two weight scales
  const uint32_t smem_base = lds_addr(smem);
  const uint32_t lo_off = l16 * kBK + (((2 * lg) ^ fx) << 4);
  const uint32_t hi_off = l16 * kBK + (((2 * lg + 1) ^ fx) << 4);
  const uint32_t scale_base = smem_base + narrow_scale_off(P);
  const uint32_t sa_lane = l16 * 4;                              // + buffer + kt*256 + 64*i
  const uint32_t sb_wave = kNarrowWsOff + wave * 2 * kNarrowMaxSteps * 4;  // + buffer + h*256 + kt*4
  const uint32_t gidx_wave = lds_addr(gidx) + 256 * wave;
  const uint32_t q_addr = lds_addr(s_q);

  // weight-scale staging: lane l fetches K block min(l, k_steps-1) of the first
  // (gate) and of the second (up) block row of this wave's columns
  const int ws_voff0 = min(lane, k_steps - 1) * 4;
  const int ws_voff1 = ws_voff0 + (kSilu ? (p.n_out / kGroup) * k_steps * 4 : 0);
  const int kstride = p.b_packed ? (p.nb / kBN) * kTileBytes : kBK;

  // per-item state of the load side: uniform descriptors, and the lane's
  // A-row and A-scale offsets
  struct Load {
    i32x4 wsrd, ssrd;
    int a_voff, as_voff;
  };
  // per-item state of the compute side
  struct Item {
    int row0, valid, nt, mf, buf;  // buf: which scale buffer holds its scales
  };

  // uniform part of item `it` (scalar loads); with a row gather, the DMA of
  // the segment's 64 gathered row indices into this wave's LDS slot
  auto decode_head = [&](int it, Load& L, Item& C) {
    const int m = it / p.n_tiles;
    const int nt = it - m * p.n_tiles;
    const int entry = first + m;
    const int e = sload_i32(p.mtile_list, 2 * entry);
    const int row0 = sload_i32(p.mtile_list, 2 * entry + 1);
    const int valid = min(kNarrowRows, sload_i32(p.offsets, e + 1) - row0);
    C.row0 = row0;
    C.valid = valid;
    C.nt = nt;
    C.mf = (valid + 15) >> 4;
    if (p.b_packed) {
      L.wsrd = make_srd(p.b + static_cast<int64_t>(e) * p.nb * p.K + static_cast<int64_t>(nt) * kTileBytes,
                        static_cast<uint32_t>(static_cast<int64_t>(p.nb) * p.K - static_cast<int64_t>(nt) * kTileBytes));
    } else {
      const int nbase = kSilu ? nt * 128 : nt * kBN;
      L.wsrd = make_srd(p.b + (static_cast<int64_t>(e) * p.nb + nbase) * p.K,
                        static_cast<uint32_t>(p.nb - nbase) * p.K);
    }
    const int nb0 = kSilu ? nt : 2 * nt + (wave >> 2);
    L.ssrd = make_srd(p.b_scale + e * kb_per_expert + static_cast<int64_t>(nb0) * k_steps,
                      static_cast<uint32_t>((kb_per_expert - static_cast<int64_t>(nb0) * k_steps) * 4));
    if (p.a_gather) load_lds_4B(g_srd, gidx + 64 * wave, (row0 + min(lane, valid - 1)) * 4, 0);
  };
  // lane offsets of item C, once its gathered row indices are in LDS
  auto decode_tail = [&](Load& L, const Item& C) {
    const int ra = min(ld_row, C.valid - 1), rs = min(lane, C.valid - 1);
    int ta = C.row0 + ra, ts = C.row0 + rs;
    if (p.a_gather) {
      ta = lds_read_i32(gidx_wave + 4 * ra) / p.gather_div;
      ts = lds_read_i32(gidx_wave + 4 * rs) / p.gather_div;
    }
    L.a_voff = buf_off(ta, p.K, ld_chunk * 16);
    L.as_voff = static_cast<int>(ts * p.as_rs) * 4;
  };

  // all K steps' activation and weight scales of item C into its buffer (wave w
  // fetches the activation scales of K steps w, w+8, ... and its own weight scales)
  auto stage_scales = [&](const Load& L, const Item& C) {
    uint8_t* sb = smem + narrow_scale_off(P) + C.buf * kNarrowScaleBuf;
    for (int kt = wave; kt < k_steps; kt += 8)
      load_lds_4B(as_srd, sb + kt * (kNarrowRows * 4), L.as_voff, static_cast<int>(kt * p.as_ks) * 4);
    i32x4 ssrd;
    ssrd.x = __builtin_amdgcn_readfirstlane(L.ssrd.x);
    ssrd.y = __builtin_amdgcn_readfirstlane(L.ssrd.y);
    ssrd.z = __builtin_amdgcn_readfirstlane(L.ssrd.z);
    ssrd.w = __builtin_amdgcn_readfirstlane(L.ssrd.w);
    uint8_t* wsb = sb + kNarrowWsOff + wave * 2 * kNarrowMaxSteps * 4;
    load_lds_4B(ssrd, wsb, ws_voff0, 0);
    load_lds_4B(ssrd, wsb + kNarrowMaxSteps * 4, ws_voff1, 0);
  };

  // the 5 loads of K step kt into ring slot `slot` and weight registers wr
  auto issue = [&](const Load& L, int kt, int slot, i32x8 (&wr)[2]) {
    // descriptors and K offsets are wave-uniform: keep them in SGPRs (a
    // descriptor in VGPRs would turn every load into a waterfall loop)
    i32x4 srd;
    srd.x = __builtin_amdgcn_readfirstlane(L.wsrd.x);
    srd.y = __builtin_amdgcn_readfirstlane(L.wsrd.y);
    srd.z = __builtin_amdgcn_readfirstlane(L.wsrd.z);
    srd.w = __builtin_amdgcn_readfirstlane(L.wsrd.w);
    const int ktu = __builtin_amdgcn_readfirstlane(kt);
    uint8_t* st = smem + __builtin_amdgcn_readfirstlane(slot) * kNarrowStage;
    load_lds_16B(a_srd, st + 8 * wave * kBK, L.a_voff, ktu * kBK);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      // weights are read once: non-temporal loads keep them from displacing
      // the 256x256 kernel's operand panels in the XCD's L2
      wr[j].lo = hk_raw_buffer_load_v4i32(srd, wvoff[2 * j], ktu * kstride, kAuxNT);
      wr[j].hi = hk_raw_buffer_load_v4i32(srd, wvoff[2 * j + 1], ktu * kstride, kAuxNT);
    }
  };

  // ---- first item --------------------------------------------------------
  // Items come from one atomic counter, so workgroups that start late (their
  // CUs were busy) simply take fewer.  Thread 0 fetches the index after next
  // as soon as it publishes one; its result is first needed an item later.
  // Beside 256x256 tiles only narrow_active workgroups take items: the first
  // ones to start (an atomic slot counter), wherever the hardware placed them;
  // later ones exit and leave their CUs to the 256x256 kernel.
  const bool limited = first > 0 && p.narrow_active > 0;
  int nxt = 0;
  if (tid == 0) {
    int it0 = n_items;  // "no item": exit
    if (!limited || atomicAdd(item_ctr + 2, 1) < p.narrow_active) {
      it0 = atomicAdd(item_ctr, 1);
      nxt = atomicAdd(item_ctr, 1);
    }
    lds_write_i32(q_addr, it0);
  }
  lds_barrier();
  const int it_first = __builtin_amdgcn_readfirstlane(lds_read_i32(q_addr));
  lds_barrier();  // every wave has read the slot before it is rewritten
  if (it_first >= n_items) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  Load L, Ln;
  Item C, Cn;
  C.buf = 0;
  decode_head(it_first, L, C);
  if (p.a_gather) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // own gather DMA
  decode_tail(L, C);
  stage_scales(L, C);
  i32x8 wbuf[P][2];
#pragma unroll
  for (int s = 0; s < P; ++s) issue(L, s, s, wbuf[s]);

  // The next item is decoded at the first step of group `dgroup`, at least P
  // steps before its first loads are issued (in the last group) when an item
  // has two or more groups; its gathered row indices have landed by then.
  const int dgroup = groups >= 2 ? groups - 2 : 0;
  int cp_slot = 0;  // ring slot of the step being computed
  bool have_next = false;

  while (true) {
    constexpr int MF = 4;
    const int mf = C.mf;
    f32x4 acc[MF][2];
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      acc[i][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int g = 0; g < groups; ++g) {
      const bool last_group = (g == groups - 1);
      if (g == dgroup && tid == 0) lds_write_i32(q_addr, nxt);  // read after the barrier below
#pragma unroll
      for (int s = 0; s < P; ++s) {
        const int kt = g * P + s;
        // scheduling barriers keep each step's MFMAs and loads inside the step,
        // so the operands of one step are live at a time
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_barrier<kNarrowVmPerStep * (P - 1)>();
        __builtin_amdgcn_sched_barrier(0);
        if (s == 0 && g == dgroup) {
          const int it = __builtin_amdgcn_readfirstlane(lds_read_i32(q_addr));
          have_next = it < n_items;
          if (have_next) {
            Cn.buf = C.buf ^ 1;
            decode_head(it, Ln, Cn);
            if (tid == 0) nxt = atomicAdd(item_ctr, 1);
          } else {
            Ln = L;
            Cn = C;
          }
        }
        if (s == 0 && last_group && have_next) {
          // a single-group item decodes and reads its indices in one step
          if (groups == 1 && p.a_gather) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
          decode_tail(Ln, Cn);
          stage_scales(Ln, Cn);
        }
        const uint32_t st = smem_base + __builtin_amdgcn_readfirstlane(cp_slot) * kNarrowStage;
        const uint32_t sbuf = scale_base + C.buf * kNarrowScaleBuf;
        const uint32_t sa_addr = sbuf + kt * (kNarrowRows * 4) + sa_lane;
        const float2 sbv = lds_read_w2(sbuf + sb_wave + kt * 4);
        const float sb_cur0 = sbv.x;                   // lane 0's DMA: gate / only block
        const float sb_cur1 = kSilu ? sbv.y : sbv.x;   // lane 1's DMA: up block
        // MFMAs from zero folded in with the block's scale product, in the
        // 256x256 kernel's arithmetic (fold_block)
        // fragment i (rows 16i..16i+15) only while the segment reaches it
        auto frag_step = [&](auto i_tag) {
          constexpr int i = decltype(i_tag)::value;
          i32x8 af;
          float sa_cur;
          lds_frag<2048 * i, 64 * i>(st + lo_off, st + hi_off, sa_addr, af, sa_cur);
          const float f0 = sa_cur * sb_cur0;
          const float f1 = kSilu ? sa_cur * sb_cur1 : f0;
          const f32x4 p0 = mfma_e4m3_16x16x128(wbuf[s][0], af, f32x4{0.f, 0.f, 0.f, 0.f});
          const f32x4 p1 = mfma_e4m3_16x16x128(wbuf[s][1], af, f32x4{0.f, 0.f, 0.f, 0.f});
          fold_block(acc[i][0], p0, f0);
          fold_block(acc[i][1], p1, f1);
          // each fragment's products are folded before the next fragment's LDS
          // reads (an empty volatile asm that takes the accumulators): the
          // kernel's VGPRs hold the weight prefetch window, and MFMA
          // temporaries sunk past the next fragments would spill it
          asm volatile("" : "+v"(acc[i][0]), "+v"(acc[i][1]));
        };
        frag_step(std::integral_constant<int, 0>{});
        if (mf > 1) frag_step(std::integral_constant<int, 1>{});
        if (mf > 2) frag_step(std::integral_constant<int, 2>{});
        if (mf > 3) frag_step(std::integral_constant<int, 3>{});
        __builtin_amdgcn_sched_barrier(0);
        // loads P steps ahead: this item's step kt+P, or the next item's step s
        const int ld_slot = cp_slot == 0 ? P : cp_slot - 1;
        Load LL;
        LL.wsrd = last_group ? Ln.wsrd : L.wsrd;
        LL.a_voff = last_group ? Ln.a_voff : L.a_voff;
        issue(LL, last_group ? s : kt + P, ld_slot, wbuf[s]);
        cp_slot = cp_slot == P ? 0 : cp_slot + 1;
      }
    }

    // ---- epilogue (the next item's first P steps are in flight) ----------
    // the accumulators hold the block-scaled sums
    if constexpr (!kSilu) {
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const int r = 16 * i + l16;
        if (i < mf && r < C.valid) {
          uint16_t* yrow = static_cast<uint16_t*>(p.c) + static_cast<int64_t>(C.row0 + r) * p.n_out +
                           C.nt * kBN + 32 * wave + 4 * lg;
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            uint2 v;
            v.x = pack_bf16x2(acc[i][j][0], acc[i][j][1]);
            v.y = pack_bf16x2(acc[i][j][2], acc[i][j][3]);
            st_nt8(yrow + 16 * j, v);  // not read again by this kernel
          }
        }
      }
    } else {
      // h = bf16(SiLU(gate) * up) staged in LDS, then the row's 128 columns
      // (one 1x128 group) requantised to e4m3 with their scale
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        if (i >= mf) break;
        float hv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) hv[q] = silu(acc[i][0][q]) * acc[i][1][q];
        uint2 v;
        v.x = pack_bf16x2(hv[0], hv[1]);
        v.y = pack_bf16x2(hv[2], hv[3]);
        lds_write_b64(lds_addr(ct + (16 * i + l16) * kNarrowCtLd + 16 * wave + 4 * lg), v);
      }
      lds_barrier();
      // The valid rows' 128 columns (one 1x128 group each) requantised to
      // e4m3: 16 lanes per row, 8 columns each, the row maximum by shuffles
      // within the 16 lanes; a 10-row segment keeps 160 lanes busy instead of 20.
      for (int base = 0; base < 16 * C.valid; base += kThreads) {
        const int idx = base + tid, r = idx >> 4, q = idx & 15;
        const bool live = r < C.valid;
        uint4 hv = uint4{0u, 0u, 0u, 0u};
        if (live) hv = lds_read_u4(lds_addr(ct + r * kNarrowCtLd + q * 8));
        const uint32_t w[4] = {hv.x, hv.y, hv.z, hv.w};
        float m = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u)
          m = fmaxf(m, fmaxf(fabsf(bf16_bits_to_f32(w[u] & 0xffffu)), fabsf(bf16_bits_to_f32(w[u] >> 16))));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        if (live) {
          const float sc = scale_from_amax(m);
          const QuotScale qs = quot_scale(sc);
          uint32_t qw[2];
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const uint32_t lo = w[2 * h2], hi = w[2 * h2 + 1];
            qw[h2] = pack_e4m3x4(quot_e4m3(bf16_bits_to_f32(lo & 0xffffu), qs),
                                 quot_e4m3(bf16_bits_to_f32(lo >> 16), qs),
                                 quot_e4m3(bf16_bits_to_f32(hi & 0xffffu), qs),
                                 quot_e4m3(bf16_bits_to_f32(hi >> 16), qs));
          }
          uint8_t* dst = static_cast<uint8_t*>(p.c) + static_cast<int64_t>(C.row0 + r) * p.n_out + C.nt * 128 + q * 8;
          st_nt8(dst, uint2{qw[0], qw[1]});
          if (q == 0) p.c_scale[static_cast<int64_t>(C.nt) * p.rows + C.row0 + r] = sc;
        }
      }
      // the staging tile is next written after at least P more barriers
    }
    if (!have_next) break;
    L = Ln;
    C = Cn;
  }
  // the re-loads issued after the last item land before the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace hkmoe
