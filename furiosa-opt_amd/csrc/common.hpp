// Shared host/device helpers for the gfx950 kernels: the reference numeric model (bf16 rules,
// fixed point), fast 32-bit division for odometer walks, and the wheel descriptor kernels take
// by value.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fo {

#define FO_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------------------------------------
// bf16 rules of furiosa-opt-std/src/float/bf16.rs:16-40 (bit exact).
// ---------------------------------------------------------------------------------------------

FO_HD uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
FO_HD float bits_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// Both conversions are written as selects, not branches, so per-element use compiles to
// v_cndmask instead of divergent exec-mask regions.
// bf16 -> f32 (bf16_to_f32): NaN -> 0x7fc00000, subnormal (and zero) -> signed zero.
FO_HD float bf16_to_f32(uint16_t h) {
  uint32_t w = (uint32_t)h << 16;
  uint32_t e = w & 0x7f800000u;
  w = (e == 0) ? (w & 0x80000000u) : w;
  w = ((w & 0x7fffffffu) > 0x7f800000u) ? 0x7fc00000u : w;
  return bits_f32(w);
}

// f32 -> bf16 (f32_to_bf16): NaN -> 0x7fc0, subnormal -> signed zero, else round to nearest even
// (half 2.7.1 bf16::from_f32).
FO_HD uint16_t f32_to_bf16(float f) {
  uint32_t x = f32_bits(f);
  uint32_t r = (x + 0x7fffu + ((x >> 16) & 1u)) >> 16;
  r = ((x & 0x7f800000u) == 0) ? ((x >> 16) & 0x8000u) : r;
  r = ((x & 0x7fffffffu) > 0x7f800000u) ? 0x7fc0u : r;
  return (uint16_t)r;
}

// Two f32 -> bf16 packed (a low, b high) by f32_to_bf16's rule: the hardware's round-to-nearest-even
// pair conversion (v_cvt_pk_bf16_f32), which agrees with the rule on every normal, zero and
// infinite input; when some lane of the wave holds a NaN or a subnormal (class mask 0x93: both NaNs
// and both denormal classes), those lanes take the rule element by element.
__device__ __forceinline__ uint32_t pack_bf16_rule(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass parses device code without the device builtins
  typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f2_t;
  typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 h2_t;
  uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2_t{a, b}, h2_t));
  const bool sp = __builtin_amdgcn_classf(a, 0x93) || __builtin_amdgcn_classf(b, 0x93);
  if (__builtin_expect(__any(sp), 0)) {
    if (sp) w = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  }
  return w;
#else
  return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
#endif
}

// bf16 + bf16 as `half`'s arithmetic does it: widen exactly, add in f32, round to nearest even
// (no flush: half's from_f32 keeps subnormals).
FO_HD uint16_t half_round_bf16(float f) {
  uint32_t x = f32_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
  uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}
FO_HD float half_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// ---------------------------------------------------------------------------------------------
// 8-bit floats (furiosa-opt-std/src/float/f8e4.rs, f8e5.rs), bit exact.
//
// f8e4m3: sign, 4-bit exponent (bias 7), 3-bit mantissa; no infinities, S.1111.111 is NaN, the
// largest finite value is 448 (0x7e); exponent 0 holds the subnormals m * 2^-9.
// f8e5m2: IEEE-like: bias 15, exponent 31 is inf (mantissa 0) / NaN; subnormals m * 2^-16.
// ---------------------------------------------------------------------------------------------

// Decode (f8_e4_to_f32): both NaN codes decode to the positive quiet NaN 0x7fc00000.
FO_HD float f8e4m3_to_f32(uint32_t c) {
  const uint32_t s = (c & 0x80u) << 24, e = (c >> 3) & 15u, m = c & 7u;
  if (e == 15u && m == 7u) return bits_f32(0x7fc00000u);
  if (e == 0u) return bits_f32(f32_bits((float)m * 0x1p-9f) | s);
  return bits_f32(s | ((e + 120u) << 23) | (m << 20));
}

// Encode (f8_e4_from_f32): round to nearest, ties to even, saturating at +-448 (infinities too);
// NaN -> 0x7f. Magnitudes from 2^-6 up round on the f32 bit pattern (the exponent carries into
// the code); below, the value in units of 2^-9 rounds to an integer 0..8 (8 is the code of 2^-6).
FO_HD uint8_t f32_to_f8e4m3(float v) {
  const uint32_t x = f32_bits(v), a = x & 0x7fffffffu, s = (x >> 24) & 0x80u;
  if (a > 0x7f800000u) return 0x7f;
  uint32_t code;
  if (a >= 0x3c800000u) {
    code = ((a + 0x7ffffu + ((a >> 20) & 1u)) >> 20) - (120u << 3);
    code = code > 0x7eu ? 0x7eu : code;
  } else {
    code = (uint32_t)rintf(bits_f32(a) * 512.0f);
  }
  return (uint8_t)(s | code);
}

// Decode (f8_e5_to_f32): NaN keeps its sign (-NaN for 0xfd..0xff).
FO_HD float f8e5m2_to_f32(uint32_t c) {
  const uint32_t s = (c & 0x80u) << 24, e = (c >> 2) & 31u, m = c & 3u;
  if (e == 31u) return bits_f32(s | (m ? 0x7fc00000u : 0x7f800000u));
  if (e == 0u) return bits_f32(f32_bits((float)m * 0x1p-16f) | s);
  return bits_f32(s | ((e + 112u) << 23) | (m << 21));
}

// Encode (f8_e5_from_f32): NaN -> 0x7e; |v| >= 2^16 (after rounding) -> signed inf 0x7c.
// Normal results round half away from zero on the f32 bit pattern (bit 20 decides, the exponent
// carries). Below 2^-14 the value in units of 2^-16 rounds half away from zero and is capped at
// 3, so [3.5, 4) * 2^-16 gives 3, not the smallest normal (f8e5.rs:51-54 clamps with min(3)).
FO_HD uint8_t f32_to_f8e5m2(float v) {
  const uint32_t x = f32_bits(v), a = x & 0x7fffffffu, s = (x >> 24) & 0x80u;
  if (a > 0x7f800000u) return 0x7e;
  if (a >= 0x38800000u) {  // 2^-14
    uint32_t code = ((a >> 21) - (112u << 2)) + ((a >> 20) & 1u);
    return (uint8_t)(s | (code > 0x7cu ? 0x7cu : code));
  }
  const float q = bits_f32(a) * 65536.0f;
  float t = truncf(q);
  t += (q - t >= 0.5f) ? 1.0f : 0.0f;
  return (uint8_t)(s | (t > 3.0f ? 3u : (uint32_t)t));
}

// fixedpoint_to_float (float/mod.rs:36-62): i32 with `int_width` integer bits -> f32, round to
// nearest even on the 24-bit mantissa.
FO_HD float fixedpoint_to_float(int32_t input, uint32_t int_width) {
  uint32_t absv = input < 0 ? (uint32_t)0 - (uint32_t)input : (uint32_t)input;
  uint32_t masked = absv & 0x7fffffffu;
  uint32_t lz = (masked == 0 ? 32u : (uint32_t)__builtin_clz(masked)) - 1u;
  uint32_t aligned = absv << lz;
  // round_to_nearest_even(aligned, 31, 24)
  uint32_t valid = aligned & 0x7fffffffu;
  const uint32_t shift = 31u - 24u - 2u;
  uint32_t sticky = (valid & ((1u << shift) - 1u)) != 0u;
  uint32_t interest = valid >> shift;
  uint32_t rf = ((interest & 7u) << 1) | sticky;
  uint32_t up = (rf == 6u || rf == 14u || rf == 5u || rf == 13u || rf == 7u || rf == 15u || rf == 12u) ? 1u : 0u;
  uint32_t rounded = (interest >> 2) + up;
  uint32_t mant = rounded & ((1u << 23) - 1u);
  uint32_t sign = input < 0 ? 1u : 0u;
  uint32_t expo;
  if (input == INT32_MIN) {
    expo = int_width + 127u;
  } else if (lz == 31u) {
    expo = 0u;
  } else {
    expo = int_width + 126u - lz;
    if ((rounded >> 24) != 0u) expo += 1u;
  }
  return bits_f32((sign << 31) | ((expo & 0xffu) << 23) | mant);
}

// Correctly rounded f32 square root (what Rust's f32::sqrt returns). The hardware square root is
// faithful, not correctly rounded, so the candidate is fixed up exactly: r is correct iff
// (r - ulp/2)^2 <= x <= (r + ulp/2)^2, and those squares are exact in f64 (2 x 25 bits < 53).
// A square root of an f32 is never a rounding midpoint, so no tie case exists.
FO_HD float sqrt_rn(float x) {
  if (!(x > 0.0f) || x == __builtin_inff()) return __builtin_sqrtf(x);  // 0, negative, NaN, inf
  float r = (float)__builtin_sqrt((double)x);
  uint32_t rb = f32_bits(r);
  double half = (double)(bits_f32(rb + 1) - r) * 0.5;  // half ulp above r
  double xd = (double)x;
  double hi = (double)r + half;
  double lo_half = (double)(r - bits_f32(rb - 1)) * 0.5;  // half ulp below r (smaller at a binade edge)
  double lo = (double)r - lo_half;
  if (lo * lo > xd) return bits_f32(rb - 1);
  if (hi * hi < xd) return bits_f32(rb + 1);
  return r;
}

// Correctly rounded a / r given y = RN(1/r) (Markstein's theorem: q = RN(a y) is within an ulp,
// the remainder a - q r is exact under FMA, and one FMA correction rounds correctly). Valid for
// normal operands and a normal, finite quotient.
FO_HD float div_cr(float a, float r, float y) {
  float q = a * y;
  float e = __builtin_fmaf(-q, r, a);
  return __builtin_fmaf(e, y, q);
}

// float_to_fixedpoint (float/mod.rs:22-34): round half away from zero (f64::round), clamp.
FO_HD int32_t float_to_fixedpoint(float input, uint32_t int_width) {
  if (input != input) return (f32_bits(input) >> 31) ? INT32_MIN : INT32_MAX;
  double v = (double)input * (double)(1ull << (31u - int_width));
  double r = v < 0 ? -__builtin_floor(-v + 0.5) : __builtin_floor(v + 0.5);
  if (r < -2147483648.0) r = -2147483648.0;
  if (r > 2147483647.0) r = 2147483647.0;
  return (int32_t)r;
}

// ---------------------------------------------------------------------------------------------
// 32-bit fast divmod (round-up multiply-shift, Granlund-Montgomery / Hacker's Delight 10-9).
// Valid for dividends < 2^31 and divisors >= 1.
// ---------------------------------------------------------------------------------------------
struct FastDiv {
  uint32_t d = 1, m = 0, s = 0;
  FastDiv() = default;
  explicit FastDiv(uint32_t div) : d(div) {
    // l = ceil(log2 d); m = floor(2^32 (2^l - d) / d) + 1; n / d = (mulhi(n, m) + n) >> l.
    uint32_t l = 0;
    while ((1ull << l) < div) ++l;
    m = (uint32_t)((((1ull << l) - div) << 32) / div + 1);
    s = l;
  }
  FO_HD uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t t = __umulhi(n, m);
#else
    uint32_t t = (uint32_t)(((uint64_t)n * m) >> 32);
#endif
    return (uint32_t)(((uint64_t)t + n) >> s);
  }
};

// Odometer wheels as a kernel argument (innermost first). `stride[k][i]` is the stride of wheel i
// in memory k.
constexpr int kMaxWheels = 12;
template <int NMEM>
struct Wheels {
  int32_t n = 0;
  uint32_t size[kMaxWheels];
  uint32_t live[kMaxWheels];
  FastDiv div[kMaxWheels];
  int64_t stride[NMEM][kMaxWheels];
};

}  // namespace fo
