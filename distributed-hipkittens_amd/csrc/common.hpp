// Device-side building blocks for the gfx950 FP8 MoE path.
//
// Everything here is written for CDNA4 (gfx950) only: 64-lane waves, the
// v_mfma_f32_16x16x128_f8f6f4 matrix instruction, buffer loads that write
// straight into LDS (buffer_load_dwordx4 ... lds) and OCP e4m3fn FP8.
//
// Reference counterparts (behaviour only, nothing is shared):
//   fp8 MFMA wrapper      include/cdna4/ops/warp/register/tile/mma.cuh:97-125
//   buffer resource       include/cdna4/ops/warp/memory/util/util.cuh:72-88
//   direct global->LDS    include/cdna4/ops/warp/memory/util/util.cuh:117-124
//   bf16 RNE pack         include/cdna4/common/base_types.cuh:350-358
//   fp8 convert (SATFINITE RNE) include/cdna4/common/base_types.cuh:423-432
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hkmoe {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define HK_LDS __attribute__((address_space(3)))

constexpr int kWave = 64;
constexpr int kGroup = 128;  // K-block / scale group width

// ---------------------------------------------------------------------------
// buffer resources and direct global->LDS loads
// ---------------------------------------------------------------------------
extern "C" __device__ void hk_raw_buffer_load_lds(i32x4 rsrc, HK_LDS uint32_t* lds_base, int size,
                                                  int voffset, int soffset, int offset,
                                                  int aux) __asm("llvm.amdgcn.raw.buffer.load.lds");

// 128-bit buffer descriptor: base address, stride 0, num_records = bytes that
// may be read (offsets past it read as zero), raw untyped dword access.
__device__ __forceinline__ i32x4 make_srd(const void* base, uint32_t num_bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  i32x4 r;
  r.x = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(p & 0xffffffffu));
  r.y = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(p >> 32));
  r.z = __builtin_amdgcn_readfirstlane(static_cast<int32_t>(num_bytes));
  r.w = 0x00020000;
  return r;
}

// One wave instruction: lane i copies 16 bytes from rsrc + voffset + soffset
// into lds_base + 16*i (lds_base and soffset must be wave-uniform).
__device__ __forceinline__ void load_lds_16B(i32x4 rsrc, void* lds_base, int voffset, int soffset = 0) {
  hk_raw_buffer_load_lds(rsrc, reinterpret_cast<HK_LDS uint32_t*>(
                                   reinterpret_cast<uintptr_t>(lds_base)),
                         16, voffset, soffset, 0, 0);
}

// Same with 4 bytes per lane (lane i -> lds_base + 4*i).
__device__ __forceinline__ void load_lds_4B(i32x4 rsrc, void* lds_base, int voffset, int soffset = 0) {
  hk_raw_buffer_load_lds(rsrc, reinterpret_cast<HK_LDS uint32_t*>(
                                   reinterpret_cast<uintptr_t>(lds_base)),
                         4, voffset, soffset, 0, 0);
}

// 16 bytes loaded / stored non-temporally (data touched once: the L2 does not
// keep it at the expense of data that is reused).
__device__ __forceinline__ uint4 ld_nt16(const void* p) {
  const i32x4 v = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
  return uint4{static_cast<uint32_t>(v.x), static_cast<uint32_t>(v.y), static_cast<uint32_t>(v.z),
               static_cast<uint32_t>(v.w)};
}
__device__ __forceinline__ void st_nt8(void* p, uint2 v) {
  typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
  const i32x2 d = {static_cast<int>(v.x), static_cast<int>(v.y)};
  __builtin_nontemporal_store(d, reinterpret_cast<i32x2*>(p));
}
__device__ __forceinline__ void st_nt16(void* p, uint4 v) {
  const i32x4 d = {static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
  __builtin_nontemporal_store(d, reinterpret_cast<i32x4*>(p));
}

// Cache-policy operand of the buffer intrinsics on gfx950: bit 0 = sc0,
// bit 1 = nt (non-temporal: the line is not expected to be reused), bit 4 = sc1.
constexpr int kAuxNT = 2;

// 16-byte buffer store: lane stores `v` at rsrc + voffset; stores at offsets
// past the descriptor's num_records are dropped by the hardware, so a
// descriptor bounded at the last valid row makes a tile's row stores
// unconditional (no branch around each store).
extern "C" __device__ void hk_raw_buffer_store_v4i32(i32x4 data, i32x4 rsrc, int voffset, int soffset,
                                                     int aux) __asm("llvm.amdgcn.raw.buffer.store.v4i32");
template <int AUX = 0>
__device__ __forceinline__ void store_16B(i32x4 rsrc, int voffset, uint4 v) {
  const i32x4 d = {static_cast<int>(v.x), static_cast<int>(v.y), static_cast<int>(v.z), static_cast<int>(v.w)};
  hk_raw_buffer_store_v4i32(d, rsrc, voffset, 0, AUX);
}

__device__ __forceinline__ void wait_vmem_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Buffer offset row * stride + add in unsigned 32-bit arithmetic (the buffer
// instruction reads its offset as unsigned): operands up to 4 GiB, which the
// host checks, address correctly and without signed overflow.
__device__ __forceinline__ int buf_off(int row, int stride, int add) {
  return static_cast<int>(static_cast<uint32_t>(row) * static_cast<uint32_t>(stride) + static_cast<uint32_t>(add));
}

// ---------------------------------------------------------------------------
// MFMA: D(16x16 fp32) += A(16x128 e4m3) . B(16x128 e4m3)^T
// Lane l supplies row (l % 16) of each operand and 32 bytes of its K range;
// both operands use the same lane->K assignment, so any bijection of the 128
// K bytes onto (l / 16, byte) gives the full dot product.  Output: lane l holds
// D[4*(l/16) + r][l % 16], r = 0..3.  Zero scale operands select the unscaled
// instruction (v_mfma_f32_16x16x128_f8f6f4).
// ---------------------------------------------------------------------------
__device__ __forceinline__ f32x4 mfma_e4m3_16x16x128(const i32x8& a, const i32x8& b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// MFMA: D(32x32 fp32) += A(32x64 e4m3) . B(32x64 e4m3)^T (v_mfma_f32_32x32x64_f8f6f4,
// twice the work of the 16x16x128 form in twice its cycles).  Lane l supplies
// row (l % 32) of each operand and 32 of its 64 K bytes (the same assignment
// for both operands); output: lane l holds D[8*(r/4) + 4*(l/32) + r%4][l % 32]
// in register r = 0..15.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16 mfma_e4m3_32x32x64(const i32x8& a, const i32x8& b, f32x16 c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// number formats
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f32_bits(float x) { return __float_as_uint(x); }

// fp32 -> bf16 bits, round to nearest even.
__device__ __forceinline__ uint32_t bf16_rne_bits(float x) {
  const uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // NaN stays NaN
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Two fp32 -> two bf16 (lo in bits 0-15), round to nearest even: one
// v_cvt_pk_bf16_f32 (same bits as bf16_rne_bits for every non-NaN input).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// fp32 -> OCP e4m3fn byte: round to nearest even, saturate to +-448,
// NaN -> 0x7f | sign.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t u = f32_bits(x);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  const float af = __uint_as_float(a);
  if (af >= 448.0f) return sign | 0x7eu;
  if (af < 0.015625f) {  // below 2^-6: subnormal grid of step 2^-9
    const float m = __builtin_rintf(af * 512.0f);  // exact scaling, RNE
    return sign | static_cast<uint32_t>(m);       // m == 8 encodes 2^-6
  }
  // normal: keep 3 mantissa bits with RNE on the 20 dropped bits
  const uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
  return sign | (r - (120u << 3));  // rebias exponent 127 -> 7
}

// fl(x / s), the correctly rounded quotient that the requantisation's e4m3
// rounding starts from (the library is built with correctly rounded fp32
// division).  Multiplying by fl(1 / s) and dividing only where the product
// could round to another e4m3 value gives the same bytes, but its per-value
// test and branch cost more than the division: 26k against 20k cycles in the
// gate/up GEMM's epilogue of a 256x256 tile.
__device__ __forceinline__ float quot_e4m3(float x, float s) { return x / s; }

// The e4m3 byte of fl(x / s) computed without a division per value.  Per
// scale (QuotScale): s is brought into [1, 2) by an exact power of two 2^sh,
// and y = fl(1 / s') is its correctly rounded reciprocal.  Per value: x' = x
// 2^sh (exact: |x| <= 448 s, so x' <= 2^10), q0 = fl(x' y) is within one ulp
// of x'/s', the remainder x' - q0 s' is exact in one FMA, and fl(q0 + r y) is
// then the correctly rounded x'/s' = x/s (Markstein's theorem: P. Markstein,
// "Computation of elementary functions on the IBM RISC System/6000 processor",
// IBM J. Res. Dev. 34(1), 1990; restated in J.-M. Muller et al., Handbook of
// Floating-Point Arithmetic, 2nd ed., section 4.7).  The scaling keeps the
// remainder clear of underflow for every quotient of at least 2^-10, the
// smallest that rounds to a nonzero e4m3 value; unscaled, tiny x and s gave
// wrong corrections.  One ldexp, a product and two FMAs per value instead of
// the division's eleven dependent operations; hkmoe_requant_quotient_check
// compares the e4m3 bytes with those of x / s over every bf16 x and bf16 row
// maximum the GEMM epilogues can see.
struct QuotScale {
  float s1;  // s 2^sh, in [1, 2)
  float y;   // fl(1 / s1)
  int sh;
};
__device__ __forceinline__ QuotScale quot_scale(float s) {
  // s = +inf (a row whose h overflowed): s' = 1, y = 0, no shift give x / inf
  // exactly (q0 = 0, r = x, q = +-0; an infinite x gives NaN)
  const bool inf = __builtin_isinf(s);
  const int sh = inf ? 0 : 1 - __builtin_amdgcn_frexp_expf(s);  // s = m 2^e, m in [0.5, 1)
  const float s1 = inf ? 1.0f : __builtin_amdgcn_ldexpf(s, sh);
  return QuotScale{s1, inf ? 0.0f : 1.0f / s1, sh};
}
__device__ __forceinline__ float quot_e4m3(float x, const QuotScale& q) {
#pragma clang fp contract(off)
  const float x1 = __builtin_amdgcn_ldexpf(x, q.sh);
  const float q0 = x1 * q.y;
  const float r = __builtin_fmaf(-q0, q.s1, x1);
  // s > 0, so the quotient has x's sign; this also keeps -0 / s = -0, which
  // q0 + r*y = -0 + +0 would turn into +0
  return __builtin_copysignf(__builtin_fmaf(r, q.y, q0), x);
}

// Four finite fp32 -> four e4m3fn bytes (a in bits 0-7), round to nearest
// even, saturating at +-448: a clamp to [-448, 448] and two hardware packed
// conversions.  (The conversion alone rounds exactly like f32_to_e4m3 for
// |v| <= 448 but gives NaN above 464 instead of saturating; the clamp makes the
// two agree on every finite input.)
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
  const float lo = -448.0f, hi = 448.0f;
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(a, lo, hi),
                                          __builtin_amdgcn_fmed3f(b, lo, hi), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_amdgcn_fmed3f(c, lo, hi),
                                      __builtin_amdgcn_fmed3f(d, lo, hi), w, true);
  return static_cast<uint32_t>(w);
}

__device__ __forceinline__ float e4m3_to_f32(uint32_t q) {
  const uint32_t s = (q & 0x80u) << 24;
  const uint32_t e = (q >> 3) & 0xfu;
  const uint32_t m = q & 0x7u;
  float v;
  if (e == 0)
    v = static_cast<float>(m) * 0.001953125f;  // m * 2^-9
  else if (e == 0xf && m == 0x7)
    v = __uint_as_float(0x7fc00000u);
  else
    v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(v) | s);
}

// Scale of a quantisation group: amax / 448, floored at the smallest normal
// fp32 (2^-126) so every scale is a positive normal number; 1 for an all-zero
// group.
__device__ __forceinline__ float scale_from_amax(float amax) {
  return amax > 0.0f ? fmaxf(amax / 448.0f, 1.17549435e-38f) : 1.0f;
}

// ---------------------------------------------------------------------------
// wave reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

// The lane id computed where it is used (a volatile asm is neither hoisted nor
// shared): for code that runs once per tile in a kernel at the VGPR limit,
// where a lane constant hoisted to the kernel entry would be spilled.
__device__ __forceinline__ int lane_here() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

}  // namespace hkmoe
