// The matrix-vector form of BufStorage::contraction_in (storage/buf.rs:401-447): one lhs vector x
// [K] against the rows of w (row n at n * ldw, contiguous along k), out[n * ldo] =
// narrow(sum_k widen(x[k]) * widen(w[n, k])). This is the shape every GEMV of the transformer's
// decode step takes (projection.rs proj_q / proj_p / proj_o, mlp.rs up / gate / down, lm_head.rs):
// one token against a weight matrix.
//
// Each output cell is folded by one lane, left to right from zero in k order, with the product and
// the sum rounded separately: the emulator's fold, bit-exact. The parallelism is across cells, so a
// block stages the weight rows of its R cells through LDS with coalesced 16-byte loads from all
// of its waves (double-buffered, the next stage's loads in flight while the current one is folded)
// and the first R lanes of wave 0 fold them. R is chosen per launch so that small N still spreads
// over many CUs; the fold chain (K dependent adds per cell) then bounds a small GEMV, and HBM
// bounds a large one.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvStage = 16384;                         // weight bytes staged per block per step
constexpr int kGemvChunks = kGemvStage / 16;              // 16-byte chunks per stage
constexpr int kGemvPer = kGemvChunks / kGemvThreads;      // chunks per thread per stage

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

template <typename Out>
__device__ __forceinline__ Out narrow_out(float a);
template <>
__device__ __forceinline__ float narrow_out<float>(float a) {
  return a;
}
template <>
__device__ __forceinline__ uint16_t narrow_out<uint16_t>(float a) {
  return f32_to_bf16(a);
}

// R cells per block; KC = k elements per stage.
template <int R, typename Out>
__global__ void __launch_bounds__(kGemvThreads) k_gemv_bf16(Out* __restrict__ out, const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w, int64_t N, int64_t K,
                                                           int64_t ldw, int64_t ldo) {
  constexpr int KC = kGemvStage / (R * 2);  // k elements per stage
  constexpr int CPR = KC / 8;               // 16-byte chunks per row per stage
  constexpr int RS = KC + 8;                // LDS row stride in elements: +16 bytes spreads the fold's banks
  __shared__ __attribute__((aligned(16))) uint16_t slab[2][R * RS];
  __shared__ __attribute__((aligned(16))) float xs[2][KC];
  const int t = threadIdx.x;
  const int64_t n0 = (int64_t)blockIdx.x * R;
  const int stages = (int)((K + KC - 1) / KC);

  uint4 reg[kGemvPer];
  uint4 xreg = make_uint4(0, 0, 0, 0);
  auto load = [&](int s) {
    const int64_t k0 = (int64_t)s * KC;
#pragma unroll
    for (int u = 0; u < kGemvPer; ++u) {
      const int c = t + u * kGemvThreads;
      const int row = c / CPR, col = (c % CPR) * 8;
      const int64_t n = n0 + row, k = k0 + col;
      reg[u] = (n < N && k < K) ? *(const uint4*)(w + n * ldw + k) : make_uint4(0, 0, 0, 0);
    }
    if (t < CPR) {
      const int64_t k = k0 + t * 8;
      xreg = k < K ? *(const uint4*)(x + k) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kGemvPer; ++u) {
      const int c = t + u * kGemvThreads;
      const int row = c / CPR, col = (c % CPR) * 8;
      *(uint4*)&slab[buf][row * RS + col] = reg[u];
    }
    if (t < CPR) {
      float* d = &xs[buf][t * 8];
      *(float4*)d = make_float4(bf16_lo(xreg.x), bf16_hi(xreg.x), bf16_lo(xreg.y), bf16_hi(xreg.y));
      *(float4*)(d + 4) = make_float4(bf16_lo(xreg.z), bf16_hi(xreg.z), bf16_lo(xreg.w), bf16_hi(xreg.w));
    }
  };

  float acc = 0.0f;
  const bool folder = t < R;
  load(0);
  store(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int buf = s & 1;
    if (s + 1 < stages) load(s + 1);
    if (folder) {
      const int kc = (int)min((int64_t)KC, K - (int64_t)s * KC);  // a multiple of 8
      const uint16_t* row = &slab[buf][t * RS];
      for (int k = 0; k < kc; k += 8) {
        const uint4 wv = *(const uint4*)(row + k);
        const float4 xa = *(const float4*)&xs[buf][k];
        const float4 xb = *(const float4*)&xs[buf][k + 4];
        acc = __fadd_rn(acc, __fmul_rn(xa.x, bf16_lo(wv.x)));
        acc = __fadd_rn(acc, __fmul_rn(xa.y, bf16_hi(wv.x)));
        acc = __fadd_rn(acc, __fmul_rn(xa.z, bf16_lo(wv.y)));
        acc = __fadd_rn(acc, __fmul_rn(xa.w, bf16_hi(wv.y)));
        acc = __fadd_rn(acc, __fmul_rn(xb.x, bf16_lo(wv.z)));
        acc = __fadd_rn(acc, __fmul_rn(xb.y, bf16_hi(wv.z)));
        acc = __fadd_rn(acc, __fmul_rn(xb.z, bf16_lo(wv.w)));
        acc = __fadd_rn(acc, __fmul_rn(xb.w, bf16_hi(wv.w)));
      }
    }
    if (s + 1 < stages) store(buf ^ 1);
    __syncthreads();
  }
  if (folder && n0 + t < N) out[(n0 + t) * ldo] = narrow_out<Out>(acc);
}

template <int R>
void gemv_r(hipStream_t s, void* out, const uint16_t* x, const uint16_t* w, fo_dtype out_t, int64_t N, int64_t K,
            int64_t ldw, int64_t ldo) {
  const int64_t blocks = (N + R - 1) / R;
  if (out_t == FO_F32)
    hipLaunchKernelGGL((k_gemv_bf16<R, float>), dim3((unsigned)blocks), dim3(kGemvThreads), 0, s, (float*)out, x, w,
                       N, K, ldw, ldo);
  else
    hipLaunchKernelGGL((k_gemv_bf16<R, uint16_t>), dim3((unsigned)blocks), dim3(kGemvThreads), 0, s,
                       (uint16_t*)out, x, w, N, K, ldw, ldo);
  FO_HIP(hipGetLastError());
}

}  // namespace

bool gemv_supported(fo_dtype in_t, fo_dtype out_t, const void* x, const void* w, int64_t N, int64_t K,
                    int64_t ldw) {
  return in_t == FO_BF16 && (out_t == FO_F32 || out_t == FO_BF16) && ((uintptr_t)x % 16) == 0 &&
         ((uintptr_t)w % 16) == 0 && K > 0 && K % 8 == 0 && ldw % 8 == 0 && N > 0 && N < (1ll << 31) &&
         (N + 15) / 16 < (1ll << 31);
}

void launch_gemv(hipStream_t s, void* out, const void* x, const void* w, fo_dtype in_t, fo_dtype out_t, int64_t N,
                 int64_t K, int64_t ldw, int64_t ldo) {
  require(gemv_supported(in_t, out_t, x, w, N, K, ldw), "gemv: unsupported operands");
  const uint16_t *xp = (const uint16_t*)x, *wp = (const uint16_t*)w;
  // Rows per block: 64 where that still gives 512 blocks, else fewer so a small N spreads out.
  if (N >= 64 * 512)
    gemv_r<64>(s, out, xp, wp, out_t, N, K, ldw, ldo);
  else if (N >= 32 * 512)
    gemv_r<32>(s, out, xp, wp, out_t, N, K, ldw, ldo);
  else
    gemv_r<16>(s, out, xp, wp, out_t, N, K, ldw, ldo);
}

}  // namespace fo
