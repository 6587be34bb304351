// Device helpers for the gfx950 FP8-V decode kernels: BF16/E4M3FN conversions, DPP and
// cross-row wave reductions, MFMA operand types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sdv {

constexpr int kBlock = 16;   // tokens per page block
constexpr int kWave = 64;    // CDNA wavefront width

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- BF16
// Loads of page data that is read exactly once per call (K, V codes, V scales) carry the
// non-temporal hint: on gfx950 streaming reads with it sustain a higher share of HBM
// bandwidth than plain loads, and they do not displace the reused lines (scores, q).
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream16(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round fp32 to the nearest BF16 (ties to even) and return it as fp32 (v_cvt_pk_bf16_f32).
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ uint32_t bf16_bits(float x) {
  __bf16 h = (__bf16)x;
  return (uint32_t)__builtin_bit_cast(uint16_t, h);
}

// Two fp32 -> packed BF16 pair (round to nearest even), one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The eager score rounding bf16(bf16(x) * c) of four fp32 values, returned as fp32: the same
// round-to-nearest-even conversions as round_bf16 per value (bitwise equal), two values per
// v_cvt_pk_bf16_f32 (8 instead of 10 VALU operations per pair).
__device__ __forceinline__ void round_scaled4(float x0, float x1, float x2, float x3, float c, float (&y)[4]) {
  const uint32_t r01 = pack_bf16x2(x0, x1), r23 = pack_bf16x2(x2, x3);
  const uint32_t s01 = pack_bf16x2(bf16_lo(r01) * c, bf16_hi(r01) * c);
  const uint32_t s23 = pack_bf16x2(bf16_lo(r23) * c, bf16_hi(r23) * c);
  y[0] = bf16_lo(s01);
  y[1] = bf16_hi(s01);
  y[2] = bf16_lo(s23);
  y[3] = bf16_hi(s23);
}

// ---------------------------------------------------------------- E4M3FN
// Encode fp32 -> OCP E4M3FN code, round to nearest even; |x| > 464 (rounds past 448), Inf and
// NaN give NaN (0x7F) with the input's sign.  Integer arithmetic on the fp32 bit pattern
// for the normal range; the subnormal range (|x| < 2^-6) is rounded as RNE(|x| * 2^9), where
// the power-of-two scaling is exact and v_rndne_f32 rounds ties to even.
__device__ __forceinline__ uint32_t e4m3fn_encode(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7FFFFFFFu;
  uint32_t r;
  if (a > 0x43E80000u) {                 // > 464.0, Inf, NaN
    r = 0x7Fu;
  } else if (a >= 0x3C800000u) {         // >= 2^-6: normal E4M3
    const uint32_t t = a + 0x7FFFFu + ((a >> 20) & 1u);
    r = (t >> 20) - (120u << 3);         // fp32 exponent bias 127 -> E4M3 bias 7
  } else {
    r = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
  }
  return r | sign;
}

// E4M3FN code (low byte of `w` selected by `sel`) -> fp32, exact (v_cvt_f32_fp8, OCP on gfx950).
__device__ __forceinline__ float e4m3fn_decode(uint32_t w, int sel) {
  switch (sel) {
    case 0: return __builtin_amdgcn_cvt_f32_fp8(w, 0);
    case 1: return __builtin_amdgcn_cvt_f32_fp8(w, 1);
    case 2: return __builtin_amdgcn_cvt_f32_fp8(w, 2);
    default: return __builtin_amdgcn_cvt_f32_fp8(w, 3);
  }
}

// ---------------------------------------------------------------- V quantization
// Shared by the append kernel and the single launch's in-kernel append, so both write the
// same bytes.

// Max over the `LPR` lanes of each row (LPR = 8 or 16 consecutive lanes) of non-negative
// fp32 bit patterns (unsigned compare; NaN propagates like torch.amax).  Every lane of the
// row receives the row's maximum.
template <int LPR>
__device__ __forceinline__ uint32_t row_max_bits(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));   // quad [1,0,3,2]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));   // quad [2,3,0,1]
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));  // half-row mirror
  if (LPR == 16)
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));  // row mirror
  return v;
}

// Max-abs bit pattern of the 8 BF16 values of a 16-byte piece (sign cleared).
__device__ __forceinline__ uint32_t abs_max_bits8(uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  uint32_t mb = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    mb = max(mb, (w[i] << 16) & 0x7FFFFFFFu);
    mb = max(mb, w[i] & 0x7FFF0000u);
  }
  return mb;
}

// Smallest max-abs (fp32 bits, 2^-60) of the fast route below: from there up to the largest
// finite value, 1/s stays a normal fp32 and every intermediate that can change a code is normal.
constexpr uint32_t kFastMinAmaxBits = 0x21800000u;

// RN(x / s) from r = RN(1/s): q0 = RN(x r), e = x - s q0 (exact, one fma), RN(q0 + e r)
// (Markstein's correction step).  For s = RN(max|v| / 448) or RN(max|v| * RN(1/448)) with
// max|v| = 0 or in [2^-60, max finite], and every BF16 x with |x| <= max|v|, the E4M3FN code
// of this value equals the code of the IEEE quotient: tests/native/quotient_check.c walks all
// such (max|v|, x) pairs and finds no difference (fp32 results differ only below 2^-10, code 0).
// The sign is copied from x, as the quotient by a positive s has it (also for -0).
__device__ __forceinline__ float quotient_rn(float x, float s, float r) {
#pragma clang fp contract(off)
  const float ax = fabsf(x);
  const float q0 = ax * r;
  const float e = __builtin_fmaf(-q0, s, ax);
  return copysignf(__builtin_fmaf(e, r, q0), x);
}

// Per token: s = max|v| / 448 evaluated per scale_mode (0: IEEE division, 1: times RN(1/448)),
// s == 0 -> 1; r = RN(1/s); fast: whether quotient_rn's proof covers this max-abs (bits ab).
__device__ __forceinline__ void token_scale(uint32_t ab, int scale_mode, float& s, float& r, bool& fast) {
  const float amax = __uint_as_float(ab);
  float sc = (scale_mode == 1) ? amax * (1.0f / 448.0f) : amax / 448.0f;
  if (sc == 0.0f) sc = 1.0f;
  s = sc;
  r = 1.0f / sc;
  fast = ab == 0 || (ab >= kFastMinAmaxBits && ab < 0x7F800000u);
}

// ---------------------------------------------------------------- page slots
// Slot (block * 16 + offset) of position `pos` of a sequence, through its block-table row;
// -1 when the position lies past the row or its block id is not a valid page.
__device__ __forceinline__ int table_slot(const int32_t* bt_row, int max_blocks, int num_blocks, int pos) {
  if (pos < 0 || (pos >> 4) >= max_blocks) return -1;
  const int pb = bt_row[pos >> 4];
  return (pb >= 0 && pb < num_blocks) ? pb * kBlock + (pos & (kBlock - 1)) : -1;
}

// ---------------------------------------------------------------- wave reductions
// DPP row rotate (within each 16-lane row).
template <int N>
__device__ __forceinline__ float dpp_row_ror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
template <int N>
__device__ __forceinline__ uint32_t dpp_row_ror_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x120 + N, 0xF, 0xF, false);
}

// Max of a non-negative fp32 over all 64 lanes (unsigned compare of the bit patterns is
// monotonic for non-negative floats and propagates NaN like torch.amax).  Wave-uniform result.
__device__ __forceinline__ uint32_t wave_max_nonneg_bits(uint32_t v) {
  v = max(v, dpp_row_ror_u<8>(v));
  v = max(v, dpp_row_ror_u<4>(v));
  v = max(v, dpp_row_ror_u<2>(v));
  v = max(v, dpp_row_ror_u<1>(v));
  const uint32_t r0 = __builtin_amdgcn_readlane(v, 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(v, 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(v, 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(v, 48);
  return max(max(r0, r1), max(r2, r3));
}

// Lane exchanges without an LDS round trip.  lane_xor_low<X>: the value of lane (lane ^ X) --
// for every lane when X = 1 or 2 (quad permutes), and for the lanes whose bit X is clear when
// X = 4 or 8 (DPP row shift left: lane i reads lane i + X of its 16-lane row; the lanes past
// the row's end read 0).
template <int X>
__device__ __forceinline__ float lane_xor_low(float v) {
  static_assert(X == 1 || X == 2 || X == 4 || X == 8, "quad permutes and row shifts only");
  constexpr int ctrl = X == 1 ? 0xB1 : X == 2 ? 0x4E : X == 4 ? 0x104 : 0x108;
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, false));
}
// lane_pair<X>, X = 16 or 32: the values of the two lanes X apart that this lane belongs to,
// lower lane first (rows 2k and 2k+1 of 16 lanes, or the two halves of 32), the same pair in
// both lanes (gfx950 v_permlane16_swap / v_permlane32_swap).
template <int X>
__device__ __forceinline__ float2 lane_pair(float v) {
  static_assert(X == 16 || X == 32, "row pairs or wave halves");
  const uint32_t u = __float_as_uint(v);
  if constexpr (X == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
  }
}

// Online-softmax statistic merge: (m, l) with l = sum exp(s - m); m = -inf means empty.
__device__ __forceinline__ void merge_stat(float& m, float& l, float m2, float l2) {
  const float mn = fmaxf(m, m2);
  if (mn == -INFINITY) return;
  const float a = (m == -INFINITY) ? 0.0f : l * expf(m - mn);
  const float b = (m2 == -INFINITY) ? 0.0f : l2 * expf(m2 - mn);
  m = mn;
  l = a + b;
}

}  // namespace sdv
