// MFMA contraction for mapped operands whose rows, columns and batch cells are spread over several
// odometer wheels -- the shape the engine's own calls take. contract_outer / contract_lane
// (engine/contraction/outer/mod.rs:145-163, lane.rs:60-79) contract the layouts
// [Chip, Cluster, Slice, Time, Packet] x [Chip, Cluster, Slice, Lane, TrfElement] onto
// [Chip, Cluster, Slice, Lane, Time, Packet]: M and N split across slice, lane and time axes,
// axes both operands carry (the DM copies of a broadcast operand) act as batch cells, and padded
// axes (`1 # 2`) leave dead output cells. The fold is BufStorage::contraction_in
// (storage/buf.rs:401-447); the contracted axis must be unit-stride in both operands.
//
// Each wave computes one 32 x 32 output tile of one batch cell with the 32x32 MFMAs; each lane
// decodes its operand row (A: tile row lane % 32, B: tile column lane % 32) from the wheels with
// 32-bit magic division and reads its k-fragments straight from global memory (16 or 32 bytes per
// k-step). Rows and columns past M / N read zero and are not stored. The output cell of (m, n) is
// c_batch + c_row(m) + c_col(n); each lane stores its column's 16 cells (rows exchanged by
// shuffles). Dead output cells are zeroed by the host before the launch.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;

enum Kind { kBf16 = 0, kI8 = 1, kF8E4M3 = 2, kF8E5M2 = 3 };

// Per k-step each lane supplies FRAG bytes: k elements FRAG / EB starting at (lane / 32) * FRAG / EB.
template <int KIND>
struct Mfma;
template <>
struct Mfma<kBf16> {
  using acc_t = f32x16_t;
  using frag_t = i32x4_t;
  static constexpr int EB = 2;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  }
};
template <>
struct Mfma<kI8> {
  using acc_t = i32x16_t;
  using frag_t = i32x4_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<kF8E4M3> {
  using acc_t = f32x16_t;
  using frag_t = i32x8_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
};
template <>
struct Mfma<kF8E5M2> {
  using acc_t = f32x16_t;
  using frag_t = i32x8_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
  }
};

// OUT: 0 bf16 (from f32), 1 f32, 2 i8 (wrap), 3 i32, 5 f8e4m3, 6 f8e5m2.
template <int OUT>
struct OutT;
template <>
struct OutT<0> {
  using T = uint16_t;
  static __device__ __forceinline__ T cvt(float v) { return f32_to_bf16(v); }
};
template <>
struct OutT<1> {
  using T = float;
  static __device__ __forceinline__ T cvt(float v) { return v; }
};
template <>
struct OutT<2> {
  using T = int8_t;
  static __device__ __forceinline__ T cvt(int32_t v) { return (int8_t)v; }
};
template <>
struct OutT<3> {
  using T = int32_t;
  static __device__ __forceinline__ T cvt(int32_t v) { return v; }
};
template <>
struct OutT<5> {
  using T = uint8_t;
  static __device__ __forceinline__ T cvt(float v) { return f32_to_f8e4m3(v); }
};
template <>
struct OutT<6> {
  using T = uint8_t;
  static __device__ __forceinline__ T cvt(float v) { return f32_to_f8e5m2(v); }
};

struct WheelGemmArgs {
  const uint8_t* a;
  const uint8_t* b;
  void* c;
  int32_t M, N, K;  // K: contracted elements (unit stride in both operands)
  int32_t batches, tiles_m, tiles_n;
  Wheels<2> mw;  // row wheels (live digits): stride[0] into A, stride[1] into C
  Wheels<2> nw;  // column wheels: stride[0] into B, stride[1] into C
  Wheels<3> bw;  // batch wheels: A, B, C
};

template <int NMEM>
__device__ __forceinline__ void decode(const Wheels<NMEM>& w, uint32_t q, int64_t (&off)[NMEM]) {
#pragma unroll
  for (int k = 0; k < NMEM; ++k) off[k] = 0;
  for (int i = 0; i < w.n; ++i) {
    const uint32_t nq = w.div[i].div(q);
    const uint32_t d = q - nq * w.size[i];
#pragma unroll
    for (int k = 0; k < NMEM; ++k) off[k] += (int64_t)d * w.stride[k][i];
    q = nq;
  }
}

template <int KIND, int OUT>
__global__ void __launch_bounds__(256) k_gemm_wheels(WheelGemmArgs g) {
  using MF = Mfma<KIND>;
  using acc_t = typename MF::acc_t;
  using frag_t = typename MF::frag_t;
  using O = OutT<OUT>;
  constexpr int EB = MF::EB;
  constexpr int FRAG = (int)sizeof(frag_t);   // bytes per lane per k-step
  constexpr int KPL = FRAG / EB;              // k elements per lane per k-step
  constexpr int KSTEP = 2 * KPL;              // k elements per k-step

  const int lane = threadIdx.x & 63;
  const int64_t tile = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t per_batch = (int64_t)g.tiles_m * g.tiles_n;
  if (tile >= per_batch * g.batches) return;  // whole wave: no barrier below
  const int batch = (int)(tile / per_batch);
  const int t = (int)(tile - (int64_t)batch * per_batch);
  const int tm = t / g.tiles_n, tn = t - (t / g.tiles_n) * g.tiles_n;

  int64_t bo[3];
  decode(g.bw, (uint32_t)batch, bo);
  const int r = lane & 31, half = lane >> 5;
  const int m = tm * 32 + r, n = tn * 32 + r;
  int64_t mo[2] = {0, 0}, no[2] = {0, 0};
  const bool mok = m < g.M, nok = n < g.N;
  if (mok) decode(g.mw, (uint32_t)m, mo);
  if (nok) decode(g.nw, (uint32_t)n, no);
  const uint8_t* pa = g.a + (bo[0] + mo[0]) * EB + half * FRAG;
  const uint8_t* pb = g.b + (bo[1] + no[0]) * EB + half * FRAG;

  acc_t acc;
#pragma unroll
  for (int v = 0; v < 16; ++v) acc[v] = 0;
  for (int k0 = 0; k0 < g.K; k0 += KSTEP) {
    // The lane's k-chunk lies wholly inside or wholly past K (K is a multiple of KPL).
    const bool kin = k0 + half * KPL < g.K;
    frag_t fa, fb;
#pragma unroll
    for (int w = 0; w < FRAG / 4; ++w) fa[w] = fb[w] = 0;
    if (kin && mok) {
#pragma unroll
      for (int e = 0; e < FRAG / 16; ++e) {
        const i32x4_t q = *(const i32x4_t*)(pa + (int64_t)k0 * EB + 16 * e);
#pragma unroll
        for (int w = 0; w < 4; ++w) fa[4 * e + w] = q[w];
      }
    }
    if (kin && nok) {
#pragma unroll
      for (int e = 0; e < FRAG / 16; ++e) {
        const i32x4_t q = *(const i32x4_t*)(pb + (int64_t)k0 * EB + 16 * e);
#pragma unroll
        for (int w = 0; w < 4; ++w) fb[4 * e + w] = q[w];
      }
    }
    acc = MF::mma(fa, fb, acc);
  }

  // D[i][j]: lane holds column j = lane % 32 and rows i = 8 (v / 4) + 4 half + v % 4; every
  // lane takes part in the row-offset exchange.
  typename O::T* C = (typename O::T*)g.c;
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int i = 8 * (v / 4) + 4 * half + (v % 4);
    const int64_t crow = __shfl(mo[1], i, 64);
    const bool rok = tm * 32 + i < g.M;
    if (rok && nok) C[bo[2] + crow + no[1]] = O::cvt(acc[v]);
  }
}

__global__ void __launch_bounds__(256) k_zero_bytes(uint8_t* __restrict__ p, uint64_t n) {
  const uint64_t nv = n / 16;
  for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < nv; i += (uint64_t)gridDim.x * 256)
    ((i32x4_t*)p)[i] = i32x4_t{0, 0, 0, 0};
  for (uint64_t i = nv * 16 + (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256) p[i] = 0;
}

template <int KIND, int OUT>
void wheels_launch(hipStream_t s, const WheelGemmArgs& g) {
  const int64_t tiles = (int64_t)g.tiles_m * g.tiles_n * g.batches;
  const int64_t blocks = (tiles + 3) / 4;
  require(blocks < (1ll << 31), "gemm_wheels: too many tiles");
  hipLaunchKernelGGL((k_gemm_wheels<KIND, OUT>), dim3((unsigned)blocks), dim3(256), 0, s, g);
}

}  // namespace

void launch_zero(hipStream_t s, void* p, uint64_t bytes) {
  require(((uintptr_t)p & 15u) == 0, "zero fill: buffer must be 16-byte aligned");
  int64_t blocks = (int64_t)((bytes / 16 + 255) / 256);
  if (blocks < 1) blocks = 1;
  if (blocks > 65535ll * 16) blocks = 65535ll * 16;
  hipLaunchKernelGGL(k_zero_bytes, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t*)p, bytes);
  FO_HIP(hipGetLastError());
}

bool gemm_wheels_supported(fo_dtype in_t, fo_dtype out_t, int64_t K, int64_t elem_align) {
  const bool types = (in_t == FO_BF16 && (out_t == FO_BF16 || out_t == FO_F32)) ||
                     (in_t == FO_I8 && (out_t == FO_I8 || out_t == FO_I32)) ||
                     ((in_t == FO_F8E4M3 || in_t == FO_F8E5M2) && (out_t == in_t || out_t == FO_F32));
  // k fragments are 16-byte loads: every operand offset a lane starts from, and K, must be whole
  // fragments (8 bf16, 16 i8, 32 f8 elements).
  const int64_t kpl = in_t == FO_BF16 ? 8 : (in_t == FO_I8 ? 16 : 32);
  return types && K > 0 && K % kpl == 0 && elem_align % kpl == 0;
}

void launch_gemm_wheels(hipStream_t s, void* c, const void* a, const void* b, fo_dtype in_t, fo_dtype out_t,
                        int64_t M, int64_t N, int64_t K, int64_t batches, const Wheels<2>& mw, const Wheels<2>& nw,
                        const Wheels<3>& bw) {
  require(((uintptr_t)a & 15u) == 0 && ((uintptr_t)b & 15u) == 0, "gemm_wheels: operands must be 16-byte aligned");
  require(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31) && batches < (1ll << 31),
          "gemm_wheels: shape beyond 32-bit addressing");
  WheelGemmArgs g;
  g.a = (const uint8_t*)a;
  g.b = (const uint8_t*)b;
  g.c = c;
  g.M = (int32_t)M;
  g.N = (int32_t)N;
  g.K = (int32_t)K;
  g.batches = (int32_t)batches;
  g.tiles_m = (int32_t)((M + 31) / 32);
  g.tiles_n = (int32_t)((N + 31) / 32);
  g.mw = mw;
  g.nw = nw;
  g.bw = bw;
  if (in_t == FO_BF16 && out_t == FO_BF16)
    wheels_launch<kBf16, 0>(s, g);
  else if (in_t == FO_BF16 && out_t == FO_F32)
    wheels_launch<kBf16, 1>(s, g);
  else if (in_t == FO_I8 && out_t == FO_I8)
    wheels_launch<kI8, 2>(s, g);
  else if (in_t == FO_I8 && out_t == FO_I32)
    wheels_launch<kI8, 3>(s, g);
  else if (in_t == FO_F8E4M3 && out_t == FO_F8E4M3)
    wheels_launch<kF8E4M3, 5>(s, g);
  else if (in_t == FO_F8E4M3 && out_t == FO_F32)
    wheels_launch<kF8E4M3, 1>(s, g);
  else if (in_t == FO_F8E5M2 && out_t == FO_F8E5M2)
    wheels_launch<kF8E5M2, 6>(s, g);
  else if (in_t == FO_F8E5M2 && out_t == FO_F32)
    wheels_launch<kF8E5M2, 1>(s, g);
  else
    throw InvalidArg("gemm_wheels: unsupported dtype pair");
  FO_HIP(hipGetLastError());
}

}  // namespace fo
