// The matrix-vector form of BufStorage::contraction_in (storage/buf.rs:401-447): one lhs vector x
// [K] against the rows of w (row n at n * ldw, contiguous along k), out[n * ldo] =
// narrow(sum_k widen(x[k]) * widen(w[n, k])). This is the shape every GEMV of the transformer's
// decode step takes (projection.rs proj_q / proj_p / proj_o, mlp.rs up / gate / down, lm_head.rs):
// one token against a weight matrix.
//
// Each output cell is folded by one lane, left to right from zero in k order, with the product and
// the sum rounded separately: the emulator's fold, bit-exact. Both operands are widened by the
// reference's bf16 rule (float/bf16.rs:16-40: a subnormal reads as a signed zero); the products
// and sums themselves are IEEE f32, subnormal results included. The parallelism is across cells,
// and the chain of K dependent adds per cell bounds a small GEMV, HBM a large one. Two kernels:
//   * k_gemv_fold (K <= 4096): a block of seven waves owns 64 cells. Waves 1-6 stream the 64 weight
//     rows from HBM (16-byte loads, four stages in flight) and write the exact f32 products of each
//     96-element stage to LDS; wave 0 folds the previous stage's products, one cell per lane, so its
//     instruction stream is one LDS read per four adds. (Three producer waves left the fold waiting
//     on them; six bring a stage close to the folder's own chain of dependent adds.) The producer waves run with subnormal inputs
//     flushed and subnormal results kept (the MODE register is per wave): the reference's widen of
//     a subnormal weight to zero, then an IEEE product. The folding wave keeps full IEEE behaviour.
//   * k_gemv_bf16 (any K): R cells per block, the rows staged through LDS by all waves and folded by
//     the first R lanes of wave 0, widening each weight on the fly.
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
// The reference widen of a weight (a subnormal reads as zero; the sign of that zero cannot reach a
// fold that starts from +0, which is never -0 afterwards).
__device__ __forceinline__ float wlo(uint32_t v) { return (v & 0x7f80u) ? bf16_lo(v) : 0.0f; }
__device__ __forceinline__ float whi(uint32_t v) { return (v & 0x7f800000u) ? bf16_hi(v) : 0.0f; }

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
      const uint16_t* h = (const uint16_t*)&xreg;
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] = bf16_to_f32(h[e]);
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
        acc = __fadd_rn(acc, __fmul_rn(xa.x, wlo(wv.x)));
        acc = __fadd_rn(acc, __fmul_rn(xa.y, whi(wv.x)));
        acc = __fadd_rn(acc, __fmul_rn(xa.z, wlo(wv.y)));
        acc = __fadd_rn(acc, __fmul_rn(xa.w, whi(wv.y)));
        acc = __fadd_rn(acc, __fmul_rn(xb.x, wlo(wv.z)));
        acc = __fadd_rn(acc, __fmul_rn(xb.y, whi(wv.z)));
        acc = __fadd_rn(acc, __fmul_rn(xb.z, wlo(wv.w)));
        acc = __fadd_rn(acc, __fmul_rn(xb.w, whi(wv.w)));
      }
    }
    if (s + 1 < stages) store(buf ^ 1);
    __syncthreads();
  }
  if (folder && n0 + t < N) out[(n0 + t) * ldo] = narrow_out<Out>(acc);
}

constexpr int kFoldR = 64;                          // cells per block: one per lane of wave 0
constexpr int kFoldKC = 96;                         // k elements per stage
constexpr int kFoldCPR = kFoldKC / 8;               // 16-byte chunks per row per stage
constexpr int kFoldProducers = 384;                 // threads of waves 1-6
constexpr int kFoldPer = kFoldR * kFoldCPR / kFoldProducers;  // chunks per producer per stage (4)
constexpr int kFoldPS = kFoldKC + 4;  // product row stride in floats: 16 lanes' b128 reads cover 64 banks once
constexpr int kFoldMaxK = 4096;       // x is staged whole in LDS
constexpr int kFoldDepth = 4;         // stages of weight loads in flight per producer
static_assert(kFoldR * kFoldCPR % kFoldProducers == 0, "producer chunks must divide evenly");
// s_waitcnt lgkmcnt(0) with vmcnt and expcnt left alone: LDS traffic done, global loads still in flight.
constexpr int kWaitLds = 15 | (7 << 4) | (0 << 8) | (3 << 14);
// MODE.FP_DENORM single-precision field (bits 5:4) = 2: flush subnormal inputs, keep subnormal results.
constexpr int kModeDenormF32 = 1 | (4 << 6) | (1 << 11);  // s_setreg hwreg(HW_REG_MODE, 4, 2)
constexpr int kDenormFlushIn = 2;

// XF32: x is f32 data standing for the widen of its deferred bf16 narrow (the runtime's deferred
// casts); each element is rounded to bf16 by the narrow's rule and widened as it is staged.
template <typename Out, bool XF32>
__global__ void __launch_bounds__(64 + kFoldProducers) k_gemv_fold(Out* __restrict__ out, const void* __restrict__ x,
                                                   const uint16_t* __restrict__ w, int64_t N, int K, int64_t ldw,
                                                   int64_t ldo) {
  __shared__ __attribute__((aligned(16))) float P[2][kFoldR * kFoldPS];
  __shared__ __attribute__((aligned(16))) float xs[kFoldMaxK];
  const int t = threadIdx.x;
  const bool folder = __builtin_amdgcn_readfirstlane(t >> 6) == 0;  // wave 0 (uniform per wave)
  const int p = t - 64;
  const int64_t n0 = (int64_t)blockIdx.x * kFoldR;
  const int stages = (K + kFoldKC - 1) / kFoldKC;
  const int xchunks = K / 8;

  // Every producer issues the same loads every stage (addresses past N or K are clamped onto valid
  // data, whose products are skipped or never folded into a written cell), so the loads complete in
  // issue order and each stage waits only for its own.
  // A producer's chunks sit at fixed (row, column) places of every stage: their row pointers,
  // columns and product offsets are computed once.
  const uint16_t* wrow[kFoldPer];
  int pcol[kFoldPer], poff[kFoldPer];
#pragma unroll
  for (int u = 0; u < kFoldPer; ++u) {
    const int c = p + u * kFoldProducers;
    const int row = c / kFoldCPR;
    pcol[u] = (c % kFoldCPR) * 8;
    poff[u] = row * kFoldPS + pcol[u];
    wrow[u] = w + min(n0 + row, N - 1) * ldw;
  }
  uint4 reg[kFoldDepth][kFoldPer];
  auto load = [&](int s, uint4 (&r)[kFoldPer]) {
    const int k0 = s * kFoldKC;
    const bool full = k0 + kFoldKC <= K;  // uniform: no chunk of the stage reaches K
#pragma unroll
    for (int u = 0; u < kFoldPer; ++u) {
      const int k = k0 + pcol[u];
      r[u] = *(const uint4*)(wrow[u] + (full || k < K ? k : K - 8));
    }
  };
  if (!folder) {
    __builtin_amdgcn_s_setreg(kModeDenormF32, kDenormFlushIn);
    constexpr int kXPer = kFoldMaxK / 8 / kFoldProducers + 1;  // x chunks per producer (3)
    uint4 xv[kXPer][XF32 ? 2 : 1];
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {
      const int c = min(p + u * kFoldProducers, xchunks - 1);
      if constexpr (XF32) {
        xv[u][0] = *((const uint4*)((const float*)x + 8 * c));
        xv[u][1] = *((const uint4*)((const float*)x + 8 * c) + 1);
      } else {
        xv[u][0] = *(const uint4*)((const uint16_t*)x + 8 * c);
      }
    }
#pragma unroll
    for (int j = 0; j < kFoldDepth; ++j) load(j, reg[j]);
#pragma unroll
    for (int u = 0; u < kXPer; ++u) {  // the reference widen of x
      const int c = p + u * kFoldProducers;
      if (c < xchunks) {
        uint16_t h[8];
        if constexpr (XF32) {
          const uint32_t* f = (const uint32_t*)&xv[u][0];
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = f32_to_bf16(bits_f32(f[e]));
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = ((const uint16_t*)&xv[u][0])[e];
        }
        float4 a = make_float4(bf16_to_f32(h[0]), bf16_to_f32(h[1]), bf16_to_f32(h[2]), bf16_to_f32(h[3]));
        float4 b = make_float4(bf16_to_f32(h[4]), bf16_to_f32(h[5]), bf16_to_f32(h[6]), bf16_to_f32(h[7]));
        *(float4*)&xs[8 * c] = a;
        *(float4*)&xs[8 * c + 4] = b;
      }
    }
  }
  // Hand-over between the waves: LDS writes done, weight loads left in flight (a __syncthreads()
  // fence would also wait for those, stalling every stage on HBM latency).
  auto handover = [] {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(kWaitLds);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
  };
  handover();

  // Iteration s: the producers write stage s's products into P[s & 1] while the folder adds stage
  // s - 1's from P[(s - 1) & 1]; the barrier then hands both over. A buffer is rewritten two
  // iterations after it was written, by which time its fold has passed a barrier. Both roles run
  // the same count of iterations (stages + 1, rounded up to whole rounds of the load ring).
  const int rounds = (stages + kFoldDepth) / kFoldDepth;
  float acc = 0.0f;
  if (!folder) {
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
      for (int j = 0; j < kFoldDepth; ++j) {
        const int s = r * kFoldDepth + j;
        // The products of stage s into P[s & 1]; FULL (a constant at each inlined use) when every
        // chunk of the stage lies below K, else chunks past K write +0.
        auto produce = [&](int s, const uint4 (&r)[kFoldPer], bool FULL) __attribute__((always_inline)) {
          float* dst = P[s & 1];
          float4 xa[kFoldPer], xb[kFoldPer];
#pragma unroll
          for (int u = 0; u < kFoldPer; ++u) {  // all x reads first, then the products
            const int k = s * kFoldKC + pcol[u];
            const int kk = FULL || k < K ? k : K - 8;
            xa[u] = *(const float4*)&xs[kk];
            xb[u] = *(const float4*)&xs[kk + 4];
          }
#pragma unroll
          for (int u = 0; u < kFoldPer; ++u) {
            const uint4 v = r[u];
            float4 a = make_float4(__fmul_rn(xa[u].x, bf16_lo(v.x)), __fmul_rn(xa[u].y, bf16_hi(v.x)),
                                   __fmul_rn(xa[u].z, bf16_lo(v.y)), __fmul_rn(xa[u].w, bf16_hi(v.y)));
            float4 b = make_float4(__fmul_rn(xb[u].x, bf16_lo(v.z)), __fmul_rn(xb[u].y, bf16_hi(v.z)),
                                   __fmul_rn(xb[u].z, bf16_lo(v.w)), __fmul_rn(xb[u].w, bf16_hi(v.w)));
            if (!FULL && s * kFoldKC + pcol[u] >= K) a = b = make_float4(0.f, 0.f, 0.f, 0.f);  // past K: +0
            *(float4*)&dst[poff[u]] = a;
            *(float4*)&dst[poff[u] + 4] = b;
          }
        };
        if ((s + 1) * kFoldKC <= K)
          produce(s, reg[j], true);
        else if (s < stages)
          produce(s, reg[j], false);
        load(s + kFoldDepth, reg[j]);
        handover();
      }
    }
  } else {
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
      for (int j = 0; j < kFoldDepth; ++j) {
        const int s = r * kFoldDepth + j;
        if (s >= 1 && s <= stages) {
          // Products past K are +0, which leave the sum unchanged. The stage's row is read whole
          // before the adds (all reads in flight at once, not one read's latency per four adds).
          const float* row = &P[(s - 1) & 1][t * kFoldPS];
          float4 v[kFoldKC / 4];
#pragma unroll
          for (int i = 0; i < kFoldKC / 4; ++i) v[i] = *(const float4*)(row + 4 * i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < kFoldKC / 4; ++i) {
            acc = __fadd_rn(acc, v[i].x);
            acc = __fadd_rn(acc, v[i].y);
            acc = __fadd_rn(acc, v[i].z);
            acc = __fadd_rn(acc, v[i].w);
          }
        }
        handover();
      }
    }
  }
  if (folder && n0 + t < N) out[(n0 + t) * ldo] = narrow_out<Out>(acc);
}

template <typename Out>
void gemv_fold(hipStream_t s, Out* out, const void* x, bool x_f32, const uint16_t* w, int64_t N, int64_t K,
               int64_t ldw, int64_t ldo) {
  const int64_t blocks = (N + kFoldR - 1) / kFoldR;
  if (x_f32)
    hipLaunchKernelGGL((k_gemv_fold<Out, true>), dim3((unsigned)blocks), dim3(64 + kFoldProducers), 0, s, out, x, w,
                       N, (int)K, ldw, ldo);
  else
    hipLaunchKernelGGL((k_gemv_fold<Out, false>), dim3((unsigned)blocks), dim3(64 + kFoldProducers), 0, s, out, x, w,
                       N, (int)K, ldw, ldo);
  FO_HIP(hipGetLastError());
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

bool gemv_takes_f32_x(int64_t K) { return K <= kFoldMaxK; }

void launch_gemv(hipStream_t s, void* out, const void* x, const void* w, fo_dtype in_t, fo_dtype out_t, int64_t N,
                 int64_t K, int64_t ldw, int64_t ldo, bool x_f32) {
  require(gemv_supported(in_t, out_t, x, w, N, K, ldw), "gemv: unsupported operands");
  require(!x_f32 || gemv_takes_f32_x(K), "gemv: an f32 x through its bf16 narrow takes K <= 4096");
  const uint16_t *xp = (const uint16_t*)x, *wp = (const uint16_t*)w;
  if (K <= kFoldMaxK) {
    if (out_t == FO_F32)
      gemv_fold<float>(s, (float*)out, x, x_f32, wp, N, K, ldw, ldo);
    else
      gemv_fold<uint16_t>(s, (uint16_t*)out, x, x_f32, wp, N, K, ldw, ldo);
    return;
  }
  // Rows per block: 64 where that still gives 512 blocks, else fewer so a small N spreads out.
  if (N >= 64 * 512)
    gemv_r<64>(s, out, xp, wp, out_t, N, K, ldw, ldo);
  else if (N >= 32 * 512)
    gemv_r<32>(s, out, xp, wp, out_t, N, K, ldw, ldo);
  else
    gemv_r<16>(s, out, xp, wp, out_t, N, K, ldw, ldo);
}

}  // namespace fo
