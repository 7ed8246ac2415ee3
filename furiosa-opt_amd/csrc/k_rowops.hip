// Fused vector-engine row chain: RMSNorm then row softmax, one HBM pass (read x, write out).
// Rounding points follow the reference RMSNorm kernel (furiosa-opt-examples/src/transformer/
// kernel/rmsnorm.rs:9-78): fetch_cast bf16 -> f32; x*x (MulF with the stash) summed by the intra-
// slice reduce; fp_div by the column count; clip Add eps; Sqrt; (x * g) / r in f32; cast to bf16 at
// commit. The softmax re-fetches the committed bf16 values: max, exp(y - max), sum, divide, cast.
//
// Layout: one wave64 per row; lane l holds the 16-byte chunks c*64 + l (8 bf16 each), so every wave
// load or store is 1 KiB contiguous. The row stays packed as bf16 in registers (x, then y); the
// waves are persistent (a grid-stride loop over rows) and keep the next two rows' x in flight while
// the current one is computed, so the load stream never drains. exp(y - max) is evaluated twice
// (for the sum, then for the output) rather than held, which frees the registers the second
// prefetched row needs at two waves per SIMD. The gain is staged once per block in
// LDS as f32.
//
// Numerics. This file is compiled with f32 denormals flushed (inputs and results, sign kept),
// which is the reference's own numeric model: its bf16 widen and narrow flush every subnormal to a
// signed zero (float/bf16.rs:16-40). With that mode a bf16 -> f32 widen is a plain shift (a
// subnormal reads as zero in every later op), a subnormal result flushes before the narrow, and
// the narrow is the hardware round-to-nearest-even v_cvt_pk_bf16_f32. The one case left is a
// non-finite value (NaN payloads and inf - inf), which the reference canonicalises: a row whose
// sum of squares, gain or y is non-finite is recomputed by the exact per-element path.
//   * (x*g)/r is the correctly rounded quotient q' = RN(q + e*y), q = RN(a*y), e = a - q*r (exact,
//     one FMA), y = RN(1/r) (Markstein's correction, exact for normal operands and results);
//   * exp and the final division feed only the output's bf16 narrow, so they use the hardware exp2
//     and reciprocal (<= 2 f32 ulps; a flip of the narrow from them is a 1-ulp change);
//   * the row max is taken on f32 y: rounding to nearest is monotone, so bf16(max y) = max bf16(y).
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

// Plain widen of the low / high bf16 of a packed word (subnormals read as zero in flush mode).
__device__ __forceinline__ float lo_raw(uint32_t w) { return bits_f32(w << 16); }
__device__ __forceinline__ float hi_raw(uint32_t w) { return bits_f32(w & 0xffff0000u); }

// Round two f32 to packed bf16 with the hardware RNE convert.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// The exact per-element path (reference rules at every rounding point), for rows holding a
// non-finite value. Reads the row again from global memory.
__device__ void row_exact(uint16_t* __restrict__ orow, const uint16_t* __restrict__ xr,
                          const uint16_t* __restrict__ gain, int cols, float eps, int lane) {
  float ss = 0.f;
  for (int i = lane; i < cols; i += 64) {
    float f = bf16_to_f32(xr[i]);
    ss = __fadd_rn(ss, __fmul_rn(f, f));
  }
  ss = wave_sum(ss);
  float r = sqrt_rn(__fadd_rn(__fdiv_rn(ss, (float)cols), eps));
  float mx = -INFINITY;
  for (int i = lane; i < cols; i += 64) {
    float y = bf16_to_f32(f32_to_bf16(__fdiv_rn(__fmul_rn(bf16_to_f32(xr[i]), bf16_to_f32(gain[i])), r)));
    mx = fmaxf(mx, y);
  }
  mx = wave_max(mx);
  float s = 0.f;
  for (int i = lane; i < cols; i += 64) {
    float y = bf16_to_f32(f32_to_bf16(__fdiv_rn(__fmul_rn(bf16_to_f32(xr[i]), bf16_to_f32(gain[i])), r)));
    s += expf(__fsub_rn(y, mx));
  }
  s = wave_sum(s);
  for (int i = lane; i < cols; i += 64) {
    float y = bf16_to_f32(f32_to_bf16(__fdiv_rn(__fmul_rn(bf16_to_f32(xr[i]), bf16_to_f32(gain[i])), r)));
    orow[i] = f32_to_bf16(__fdiv_rn(expf(__fsub_rn(y, mx)), s));
  }
}

// NCH 16-byte chunks per lane: cols = NCH * 512.
template <int NCH>
__global__ void __launch_bounds__(256, 2) k_rmsnorm_softmax(uint16_t* __restrict__ out, const uint16_t* __restrict__ x,
                                                         const uint16_t* __restrict__ gain, int64_t rows, float cols_f,
                                                         float eps) {
  constexpr int cols = NCH * 512;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * 4;
  // The gain row is shared by every row: widen it once per block into LDS (reference widen rule),
  // and note whether it holds a non-finite value.
  __shared__ __attribute__((aligned(16))) float sg[cols];
  __shared__ int g_bad;
  if (threadIdx.x == 0) g_bad = 0;
  __syncthreads();
  // A gain at or above 2^120 in magnitude also takes the exact path: below it no y can overflow
  // once the row's sum of squares is finite, because |x_i| <= sqrt(ss) and r >= sqrt(ss / cols)
  // give |y_i| <= sqrt(cols) * max|g| < 2^7 * 2^120.
  int bad_local = 0;
  for (int i = threadIdx.x; i < cols; i += blockDim.x) {
    float gv = bf16_to_f32(gain[i]);
    sg[i] = gv;
    bad_local |= !(__builtin_fabsf(gv) < 0x1p120f);
  }
  if (bad_local) g_bad = 1;
  __syncthreads();
  const bool gain_bad = g_bad != 0;
  int64_t row = wave;
  if (row >= rows) return;

  i32x4_t cur[NCH], nxt[NCH], nx2[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) cur[c] = __builtin_nontemporal_load((const i32x4_t*)(x + row * cols + (c * 64 + lane) * 8));
  if (row + nwaves < rows) {
#pragma unroll
    for (int c = 0; c < NCH; ++c)
      nxt[c] = __builtin_nontemporal_load((const i32x4_t*)(x + (row + nwaves) * cols + (c * 64 + lane) * 8));
  }

  for (; row < rows; row += nwaves) {
    const int64_t nrow = row + nwaves, n2row = row + 2 * nwaves;
    if (n2row < rows) {
#pragma unroll
      for (int c = 0; c < NCH; ++c)
        nx2[c] = __builtin_nontemporal_load((const i32x4_t*)(x + n2row * cols + (c * 64 + lane) * 8));
    }
    // sum of squares: each square rounded, then added (MulF with the stash, then the Add reduce)
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t w = (uint32_t)cur[c][e];
        float a = lo_raw(w), b = hi_raw(w);
        ss += a * a;
        ss += b * b;
      }
    ss = wave_sum(ss);
    const float ms = __fadd_rn(__fdiv_rn(ss, cols_f), eps);  // fp_div, then clip Add eps
    const float r = sqrt_rn(ms);                              // FpUnaryOp::Sqrt
    const float rinv = __fdiv_rn(1.0f, r);
    // y = bf16((x * g) / r), kept packed; row max on the f32 values
    float mx = -INFINITY;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      f32x4_t g0 = *(const f32x4_t*)(sg + (c * 64 + lane) * 8);
      f32x4_t g1 = *(const f32x4_t*)(sg + (c * 64 + lane) * 8 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t w = (uint32_t)cur[c][e];
        float glo = e < 2 ? g0[2 * e] : g1[2 * e - 4];
        float ghi = e < 2 ? g0[2 * e + 1] : g1[2 * e - 3];
        float ylo = div_cr(lo_raw(w) * glo, r, rinv);
        float yhi = div_cr(hi_raw(w) * ghi, r, rinv);
        mx = fmaxf(mx, fmaxf(ylo, yhi));
        cur[c][e] = (int)pack_bf16(ylo, yhi);
      }
    }
    mx = wave_max(mx);
    uint16_t* orow = out + row * cols;
    if (!__builtin_isfinite(ss) || gain_bad) {
      row_exact(orow, x + row * cols, gain, cols, eps, lane);
    } else {
      mx = bits_f32(pack_bf16(mx, mx) << 16);  // the max of the committed bf16 values
      // softmax: e = exp(y - max) kept in f32, s = sum(e), out = bf16(e / s)
      const float L2E = 1.4426950408889634f;
      const float mxl = mx * L2E;
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t w = (uint32_t)cur[c][e];
          s += __builtin_amdgcn_exp2f(__builtin_fmaf(lo_raw(w), L2E, -mxl));
          s += __builtin_amdgcn_exp2f(__builtin_fmaf(hi_raw(w), L2E, -mxl));
        }
      s = wave_sum(s);
      const float sinv = __builtin_amdgcn_rcpf(s);
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        i32x4_t o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          uint32_t w = (uint32_t)cur[c][e];
          o[e] = (int)pack_bf16(__builtin_amdgcn_exp2f(__builtin_fmaf(lo_raw(w), L2E, -mxl)) * sinv,
                                __builtin_amdgcn_exp2f(__builtin_fmaf(hi_raw(w), L2E, -mxl)) * sinv);
        }
        __builtin_nontemporal_store(o, (i32x4_t*)(orow + (c * 64 + lane) * 8));
      }
    }
    if (nrow < rows) {
#pragma unroll
      for (int c = 0; c < NCH; ++c) {
        cur[c] = nxt[c];
        nxt[c] = nx2[c];
      }
    }
  }
}

// Any column count: the exact per-element path, one wave per row.
__global__ void __launch_bounds__(256) k_rmsnorm_softmax_any(uint16_t* __restrict__ out, const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ gain, int64_t rows, int64_t cols,
                                                             float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  row_exact(out + row * cols, x + row * cols, gain, (int)cols, eps, lane);
}

template <int NCH>
void rs_launch(hipStream_t s, uint16_t* out, const uint16_t* x, const uint16_t* g, int64_t rows, float eps) {
  // Persistent waves: exactly as many blocks as can be resident at once (occupancy x CUs), so every
  // wave starts immediately and loops over rows; never more waves than rows.
  static int64_t resident_blocks = [] {
    int dev = 0, per_cu = 1, cus = 1;
    (void)hipGetDevice(&dev);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_rmsnorm_softmax<NCH>, 256, 0) != hipSuccess ||
        per_cu < 1)
      per_cu = 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
    return (int64_t)per_cu * cus;
  }();
  int64_t blocks = (rows + 3) / 4;
  if (blocks > resident_blocks) blocks = resident_blocks;
  hipLaunchKernelGGL(k_rmsnorm_softmax<NCH>, dim3((unsigned)blocks), dim3(256), 0, s, out, x, g, rows,
                     (float)(NCH * 512), eps);
}

}  // namespace

void launch_rmsnorm_softmax(hipStream_t s, uint16_t* out, const uint16_t* x, const uint16_t* gain, int64_t rows,
                            int64_t cols, float eps) {
  require((rows + 3) / 4 < (1ll << 31), "rmsnorm_softmax: too many rows");
  require(cols < (1ll << 30), "rmsnorm_softmax: too many columns");
  bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)out % 16 == 0) && ((uintptr_t)gain % 16 == 0);
  if (aligned && cols % 512 == 0 && cols <= 8192) {
    switch (cols / 512) {
      case 1: rs_launch<1>(s, out, x, gain, rows, eps); break;
      case 2: rs_launch<2>(s, out, x, gain, rows, eps); break;
      case 4: rs_launch<4>(s, out, x, gain, rows, eps); break;
      case 8: rs_launch<8>(s, out, x, gain, rows, eps); break;
      case 16: rs_launch<16>(s, out, x, gain, rows, eps); break;
      default:
        hipLaunchKernelGGL(k_rmsnorm_softmax_any, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, out, x, gain, rows,
                           cols, eps);
    }
  } else {
    hipLaunchKernelGGL(k_rmsnorm_softmax_any, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s, out, x, gain, rows,
                       cols, eps);
  }
  FO_HIP(hipGetLastError());
}

}  // namespace fo
