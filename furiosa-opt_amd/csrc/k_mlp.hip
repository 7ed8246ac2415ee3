// The MLP classifier chain of the reference MNIST kernel (furiosa-opt-examples/src/mnist/mod.rs:
// 8-192): fc1 contraction narrowed once to bf16 (contract_lane then cast, :23-33); bias add and
// ReLU in f32 on the re-fetched bf16 values, narrowed to bf16 (:76-88); fc2 contraction narrowed
// to bf16; bias add narrowed to bf16 (:164-176); argmax with the last maximum winning ties under
// f32::total_cmp (tests/mnist_tests.rs:41-48).
//
// Latency-bound (13 MFLOP): one workgroup per batch row keeps the whole chain on chip. Each dot
// product is one thread folding k in ascending order with separate multiply/add roundings -- the
// emulator's own fold order -- so the logits match it bit for bit.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

// f32::total_cmp order as a signed integer key.
__device__ __forceinline__ int32_t total_key(float f) {
  int32_t b = (int32_t)f32_bits(f);
  return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

__global__ void __launch_bounds__(256) k_mlp(int32_t* __restrict__ pred, uint16_t* __restrict__ logits,
                                             const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                                             const uint16_t* __restrict__ b1, const uint16_t* __restrict__ w2,
                                             const uint16_t* __restrict__ b2, int32_t in_f, int32_t hidden,
                                             int32_t out_f) {
  extern __shared__ float smem[];
  float* xs = smem;            // in_f widened inputs
  float* hs = smem + in_f;     // hidden activations (bf16-rounded, widened)
  float* ys = hs + hidden;     // logits (bf16-rounded, widened)
  const int64_t b = blockIdx.x;
  for (int i = threadIdx.x; i < in_f; i += blockDim.x) xs[i] = bf16_to_f32(x[b * in_f + i]);
  __syncthreads();
  for (int h = threadIdx.x; h < hidden; h += blockDim.x) {
    const uint16_t* wr = w1 + (int64_t)h * in_f;
    float acc = 0.f;
    for (int kk = 0; kk < in_f; ++kk) acc = __fadd_rn(acc, __fmul_rn(xs[kk], bf16_to_f32(wr[kk])));
    float hv = bf16_to_f32(f32_to_bf16(acc));                  // contract_lane + cast
    float z = fmaxf(__fadd_rn(hv, bf16_to_f32(b1[h])), 0.0f);  // clip Add, clip Max 0
    hs[h] = bf16_to_f32(f32_to_bf16(z));
  }
  __syncthreads();
  for (int o = threadIdx.x; o < out_f; o += blockDim.x) {
    const uint16_t* wr = w2 + (int64_t)o * hidden;
    float acc = 0.f;
    for (int kk = 0; kk < hidden; ++kk) acc = __fadd_rn(acc, __fmul_rn(hs[kk], bf16_to_f32(wr[kk])));
    float yv = bf16_to_f32(f32_to_bf16(acc));
    uint16_t y = f32_to_bf16(__fadd_rn(yv, bf16_to_f32(b2[o])));
    ys[o] = bf16_to_f32(y);
    if (logits) logits[b * out_f + o] = y;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int best = 0;
    int32_t bk = total_key(ys[0]);
    for (int o = 1; o < out_f; ++o) {
      int32_t kk = total_key(ys[o]);
      if (kk >= bk) {  // max_by keeps the last of equal maxima
        bk = kk;
        best = o;
      }
    }
    pred[b] = best;
  }
}

// fc1 with the products taken off the critical path: waves [0, FW) fold, one thread per hidden
// unit, in ascending k (acc = RN(acc + p_k)); the other waves compute the products
// p_k = RN(x_k * w_hk) for the next KC-wide k chunk into LDS meanwhile (16-byte weight loads, 8
// products per unit of work). Same roundings in the same order as the per-thread fold, so the
// result is bit-identical; only the products run in parallel. Needs in_f % 8 == 0, 16-byte
// aligned weights, hidden <= 256 (enough producers for kUnits per chunk) and the fc2 products
// fitting the product buffer.
constexpr int kKC = 64;          // k per chunk
constexpr int kPP = kKC + 4;     // LDS row pitch in floats (16-byte rows, conflict-free b128 reads)
constexpr int kMlpThreads = 512;
constexpr int kUnits = 4;  // producer work units per chunk per thread (hidden * kKC / 8 <= kUnits * producers)
constexpr int kAhead = 2;  // chunks of weights in flight ahead of the products
constexpr int kW2Per = 4;  // fc2 weights per thread, loaded at the start (out_f * hidden <= kW2Per * threads)
// s_waitcnt immediate (gfx9 encoding): LDS/scalar count 0, vector memory and export counts left open.
constexpr int kWaitLgkm0 = 0xF | (0x7 << 4) | (0x3 << 14);

__global__ void __launch_bounds__(kMlpThreads) k_mlp_split(int32_t* __restrict__ pred, uint16_t* __restrict__ logits,
                                                           const uint16_t* __restrict__ x,
                                                           const uint16_t* __restrict__ w1,
                                                           const uint16_t* __restrict__ b1,
                                                           const uint16_t* __restrict__ w2,
                                                           const uint16_t* __restrict__ b2, int32_t in_f,
                                                           int32_t hidden, int32_t out_f) {
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
  typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int hp = (hidden + 3) / 4 * 4;
  float* xs = smem;                                  // widened inputs, in_f (padded to 4)
  float* hs = xs + (in_f + 3) / 4 * 4;               // hidden activations
  float* ys = hs + hp;                               // logits
  float* pb = ys + (out_f + 3) / 4 * 4;              // 2 x hidden x kPP products
  const int64_t b = blockIdx.x;
  const int tid = threadIdx.x;
  const int fw = (hidden + 63) / 64;                 // folder waves
  const int nprod = kMlpThreads - fw * 64;           // producer threads
  const int nchunks = (in_f + kKC - 1) / kKC;
  constexpr int G = kKC / 8;                         // 8-product groups per row per chunk
  // fc2's weights and both biases are loaded now, so their latency hides behind fc1.
  const int n2 = out_f * hidden;
  uint16_t w2r[kW2Per];
#pragma unroll
  for (int j = 0; j < kW2Per; ++j) w2r[j] = w2[min(tid + j * kMlpThreads, n2 - 1)];
  const uint16_t b1r = b1[min(tid, hidden - 1)], b2r = b2[min(tid, out_f - 1)];
  for (int i = tid; i < in_f; i += kMlpThreads) xs[i] = bf16_to_f32(x[b * in_f + i]);
  __syncthreads();
  // Producer p owns work units p, p + nprod, ... (at most kUnits): unit u is hidden row u / G,
  // 8-product group u % G of the chunk. Its weights are loaded kAhead chunks ahead, one register
  // set per chunk in flight.
  const int ptid = tid - fw * 64, units = hidden * G;
  i32x4_t wv[kAhead][kUnits];
  // Every producer issues all kUnits loads (a unit past the end reads the last group, which its
  // produce step then skips), so the loads complete in issue order and each chunk waits for its own.
  auto load = [&](int c, int set) {
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
      const int u = min(ptid + i * nprod, units - 1), h = u / G, k0 = min(c * kKC + (u % G) * 8, in_f - 8);
      wv[set][i] = *(const i32x4_t*)(w1 + (int64_t)h * in_f + k0);
    }
  };
  auto produce = [&](int c, int buf, int set) {
    float* P = pb + buf * hidden * kPP;
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
      const int u = ptid + i * nprod, h = u / G, g = u % G, k0 = c * kKC + g * 8;
      if (u >= units || k0 >= in_f) continue;  // in_f % 8 == 0: a group is whole or absent
      const f32x4_t xa = *(const f32x4_t*)(xs + k0), xb = *(const f32x4_t*)(xs + k0 + 4);
      f32x4_t p0, p1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t uw = (uint32_t)wv[set][i][e];
        const float xl = e < 2 ? xa[2 * e] : xb[2 * e - 4], xh = e < 2 ? xa[2 * e + 1] : xb[2 * e - 3];
        // The weight's bits as an f32; its subnormals read as zero through this wave's flush of
        // subnormal inputs (set below), as the reference widen has them. A NaN weight keeps its
        // payload here but makes a NaN sum, which the bf16 narrow of fc1 canonicalises.
        const float lo = __fmul_rn(xl, __uint_as_float(uw << 16));
        const float hi = __fmul_rn(xh, __uint_as_float(uw & 0xffff0000u));
        if (e < 2) {
          p0[2 * e] = lo;
          p0[2 * e + 1] = hi;
        } else {
          p1[2 * e - 4] = lo;
          p1[2 * e - 3] = hi;
        }
      }
      *(f32x4_t*)(P + h * kPP + g * 8) = p0;
      *(f32x4_t*)(P + h * kPP + g * 8 + 4) = p1;
    }
  };
  // Barrier for LDS only: the producers' weight loads for the next chunk stay in flight across
  // it (a fenced __syncthreads would drain them).
  auto lds_barrier = [&]() {
    __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
  };
  const bool folder = tid < fw * 64;
  float acc = 0.f;
  if (!folder) {
    // MODE.FP_DENORM single-precision field = 2: subnormal inputs flushed, subnormal results kept
    // (a per-wave register; the folder waves keep full IEEE behaviour).
    __builtin_amdgcn_s_setreg(1 | (4 << 6) | (1 << 11), 2);
    load(0, 0);
    if (nchunks > 1) load(1, 1);
    produce(0, 0, 0);
    if (nchunks > 2) load(2, 0);
  }
  lds_barrier();
  for (int c = 0; c < nchunks; ++c) {
    if (folder) {
      if (tid < hidden) {
        const float* P = pb + (c & 1) * hidden * kPP + tid * kPP;
        const int kn = min(kKC, in_f - c * kKC);  // a multiple of 8
        if (kn == kKC) {
          // A full chunk's row is read whole before the adds: one LDS latency per chunk rather
          // than one per four adds.
          f32x4_t v[kKC / 4];
#pragma unroll
          for (int i = 0; i < kKC / 4; ++i) v[i] = *(const f32x4_t*)(P + 4 * i);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < kKC / 4; ++i) {
            acc = __fadd_rn(acc, v[i][0]);
            acc = __fadd_rn(acc, v[i][1]);
            acc = __fadd_rn(acc, v[i][2]);
            acc = __fadd_rn(acc, v[i][3]);
          }
        } else {
          for (int k = 0; k < kn; k += 4) {
            const f32x4_t p = *(const f32x4_t*)(P + k);
            acc = __fadd_rn(acc, p[0]);
            acc = __fadd_rn(acc, p[1]);
            acc = __fadd_rn(acc, p[2]);
            acc = __fadd_rn(acc, p[3]);
          }
        }
      }
    } else if (c + 1 < nchunks) {
      // chunk c + 1's weights are in set (c + 1) % 2; that set then takes chunk c + 3
      if ((c & 1) == 0) {
        produce(c + 1, 1, 1);
        if (c + 3 < nchunks) load(c + 3, 1);
      } else {
        produce(c + 1, 0, 0);
        if (c + 3 < nchunks) load(c + 3, 0);
      }
    }
    lds_barrier();  // chunk c folded (its buffer is free); chunk c + 1 produced
  }
  if (tid < hidden) {
    float hv = bf16_to_f32(f32_to_bf16(acc));                    // contract_lane + cast
    float z = fmaxf(__fadd_rn(hv, bf16_to_f32(b1r)), 0.0f);  // clip Add, clip Max 0
    hs[tid] = bf16_to_f32(f32_to_bf16(z));
  }
  __syncthreads();
  // fc2: the out_f x hidden products in parallel into the (free) product buffer, then one
  // thread per output folds them in ascending k.
#pragma unroll
  for (int j = 0; j < kW2Per; ++j) {
    const int i = tid + j * kMlpThreads;
    if (i < n2) {
      const int o = i / hidden, kk = i % hidden;
      pb[o * hp + kk] = __fmul_rn(hs[kk], bf16_to_f32(w2r[j]));
    }
  }
  __syncthreads();
  for (int o = tid; o < out_f; o += kMlpThreads) {
    float a2 = 0.f;
    int kk = 0;
    // Runs of 32 products read before they are added, in ascending k as before.
    for (; kk + 32 <= hidden; kk += 32) {
      f32x4_t v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = *(const f32x4_t*)(pb + o * hp + kk + 4 * i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        a2 = __fadd_rn(a2, v[i][0]);
        a2 = __fadd_rn(a2, v[i][1]);
        a2 = __fadd_rn(a2, v[i][2]);
        a2 = __fadd_rn(a2, v[i][3]);
      }
    }
    for (; kk < hidden; ++kk) a2 = __fadd_rn(a2, pb[o * hp + kk]);
    float yv = bf16_to_f32(f32_to_bf16(a2));
    uint16_t y = f32_to_bf16(__fadd_rn(yv, bf16_to_f32(o == tid ? b2r : b2[o])));
    ys[o] = bf16_to_f32(y);
    if (logits) logits[b * out_f + o] = y;
  }
  __syncthreads();
  if (tid == 0) {
    int best = 0;
    int32_t bk = total_key(ys[0]);
    for (int o = 1; o < out_f; ++o) {
      int32_t kk = total_key(ys[o]);
      if (kk >= bk) {  // max_by keeps the last of equal maxima
        bk = kk;
        best = o;
      }
    }
    pred[b] = best;
  }
}

}  // namespace

void launch_mlp(hipStream_t s, int32_t* pred, uint16_t* logits, const uint16_t* x, const uint16_t* w1,
                const uint16_t* b1, const uint16_t* w2, const uint16_t* b2, int64_t batch, int64_t in_f,
                int64_t hidden, int64_t out_f) {
  require(batch < (1ll << 31), "mlp: batch too large");
  const size_t lds_split =
      (size_t)(((in_f + 3) / 4 + (hidden + 3) / 4 + (out_f + 3) / 4) * 4 + 2 * hidden * kPP) * sizeof(float);
  const int64_t producers = kMlpThreads - (hidden + 63) / 64 * 64;
  if (in_f % 8 == 0 && hidden <= 256 && hidden * (kKC / 8) <= kUnits * producers && out_f * ((hidden + 3) / 4 * 4) <= 2 * hidden * kPP &&
      out_f * hidden <= kW2Per * kMlpThreads &&
      ((uintptr_t)w1 % 16) == 0 && lds_split <= 160 * 1024) {
    static bool attr_set = false;  // dynamic LDS above 64 KiB must be opted into
    if (!attr_set) {
      FO_HIP(hipFuncSetAttribute((const void*)k_mlp_split, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr_set = true;
    }
    hipLaunchKernelGGL(k_mlp_split, dim3((unsigned)batch), dim3(kMlpThreads), lds_split, s, pred, logits, x, w1, b1, w2,
                       b2, (int32_t)in_f, (int32_t)hidden, (int32_t)out_f);
    FO_HIP(hipGetLastError());
    return;
  }
  size_t lds = (size_t)(in_f + hidden + out_f) * sizeof(float);
  require(lds <= 64 * 1024, "mlp: layer widths exceed the LDS budget");
  hipLaunchKernelGGL(k_mlp, dim3((unsigned)batch), dim3(256), lds, s, pred, logits, x, w1, b1, w2, b2, (int32_t)in_f,
                     (int32_t)hidden, (int32_t)out_f);
  FO_HIP(hipGetLastError());
}

}  // namespace fo
