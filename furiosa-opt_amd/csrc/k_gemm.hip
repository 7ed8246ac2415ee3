// MFMA contraction for the tensor-unit path: C[m, n] = sum_k A[m, k] * B[n, k], both operands
// contiguous along k (the K-major layout the mapped GEMM config resolves to: lhs m![M/8, M%8, K],
// rhs m![N, K]). The emulator's fold is BufStorage::contraction_in (storage/buf.rs:401-447):
// widen, accumulate (f32 for bf16, i32 for i8), narrow once per output cell.
//
// Tiling (gfx950, wave64): a 256-thread block owns a BM x BN tile; its 4 waves are 2 x 2, each wave
// owning (BM/2) x (BN/2) as a grid of 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16 /
// v_mfma_i32_32x32x32_i8). K advances 128 bytes per stage; stages are double-buffered in LDS with
// the next stage's global loads in flight during the current stage's MFMAs. Rows of the LDS tiles
// are padded by 16 bytes so the 16-byte fragment reads of 32 lanes hit distinct banks.
//
// Within one MFMA the hardware's k order is irrelevant: A and B fragments are loaded with the same
// k -> (lane, element) map, and the sum over k is order-free up to f32 rounding (exact for i32).
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;

constexpr int kBKB = 128;           // K bytes per stage
constexpr int kRowB = kBKB + 16;    // padded LDS row stride in bytes

template <bool IS_I8>
struct MfmaT;
template <>
struct MfmaT<false> {
  using acc_t = f32x16_t;
  static __device__ __forceinline__ acc_t mma(const i32x4_t& a, const i32x4_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  }
};
template <>
struct MfmaT<true> {
  using acc_t = i32x16_t;
  static __device__ __forceinline__ acc_t mma(const i32x4_t& a, const i32x4_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};

struct GemmArgs {
  const uint8_t* a;
  const uint8_t* b;
  void* c;
  int64_t M, N, K;  // K in elements
  int64_t lda, ldb, ldc_m, ldc_n;  // elements
  int64_t a_batch, b_batch, c_batch;
  int32_t tiles_m, tiles_n;
  const float* scale;  // OUT == 4: per-column dequant scale
  int32_t* acc_out;    // OUT == 4: optional raw i32 accumulators (row-major, ldc_m / ldc_n)
};

// OUT: 0 = bf16 (from f32), 1 = f32, 2 = i8 (wrap), 3 = i32,
//      4 = W8A8 dequant: bf16(fixedpoint_to_float(acc, 31) * scale[col]) (+ optional raw i32)
template <bool IS_I8, int OUT, int BM, int BN>
__global__ void __launch_bounds__(256) k_gemm(GemmArgs g) {
  using M = MfmaT<IS_I8>;
  using acc_t = typename M::acc_t;
  constexpr int EB = IS_I8 ? 1 : 2;  // element bytes
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_LOADS = BM * kBKB / 16 / 256;  // 16-byte loads per thread per stage
  constexpr int B_LOADS = BN * kBKB / 16 / 256;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  auto sA = [&](int buf) { return smem + buf * (BM * kRowB); };
  auto sB = [&](int buf) { return smem + 2 * BM * kRowB + buf * (BN * kRowB); };

  // Tile order: XCD-aware. Consecutive block ids go round-robin over the 8 XCDs; regroup so each
  // XCD walks a contiguous range of tiles, ordered in column groups of 8 tiles for L2 reuse.
  const int ntiles = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  int per_xcd = (ntiles + 7) / 8;
  int tile = (bid % 8) * per_xcd + bid / 8;
  if ((ntiles % 8) != 0) tile = bid;  // keep the plain order when the split is uneven
  const int group = 8;
  int gsize = group * g.tiles_n;
  int gid = tile / gsize;
  int first_m = gid * group;
  int gm = min(g.tiles_m - first_m, group);
  int tm = first_m + (tile % gsize) % gm;
  int tn = (tile % gsize) / gm;
  const int batch = blockIdx.y;

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t KB = g.K * EB;  // K in bytes

  const uint8_t* A = g.a + (g.a_batch * batch) * EB;
  const uint8_t* B = g.b + (g.b_batch * batch) * EB;

  // Global load assignment: thread t loads 16 bytes at (row = t/8 + 32*i, byte col = (t%8)*16).
  const int lr = tid >> 3, lc = (tid & 7) * 16;
  i32x4_t ra[A_LOADS], rb[B_LOADS];

  auto load_stage = [&](int64_t kb) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int64_t row = m0 + lr + 32 * i;
      int64_t col = kb + lc;
      if (row < g.M && col < KB)
        ra[i] = *(const i32x4_t*)(A + (row * g.lda) * EB + col);
      else
        ra[i] = i32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      int64_t row = n0 + lr + 32 * i;
      int64_t col = kb + lc;
      if (row < g.N && col < KB)
        rb[i] = *(const i32x4_t*)(B + (row * g.ldb) * EB + col);
      else
        rb[i] = i32x4_t{0, 0, 0, 0};
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) *(i32x4_t*)(sA(buf) + (lr + 32 * i) * kRowB + lc) = ra[i];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) *(i32x4_t*)(sB(buf) + (lr + 32 * i) * kRowB + lc) = rb[i];
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  const int nst = (int)((KB + kBKB - 1) / kBKB);
  load_stage(0);
  store_stage(0);
  __syncthreads();

  const int frow = lane & 31;          // fragment row within a 32-row tile
  const int fcol = (lane >> 5) * 16;   // byte offset of this lane's 16 bytes within a 32-byte k-step

  for (int s = 0; s < nst; ++s) {
    const int cur = s & 1;
    if (s + 1 < nst) load_stage((int64_t)(s + 1) * kBKB);
#pragma unroll
    for (int kk = 0; kk < kBKB / 32; ++kk) {
      i32x4_t fa[TM], fb[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        fa[i] = *(const i32x4_t*)(sA(cur) + (wm * WM + i * 32 + frow) * kRowB + kk * 32 + fcol);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        fb[j] = *(const i32x4_t*)(sB(cur) + (wn * WN + j * 32 + frow) * kRowB + kk * 32 + fcol);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(fa[i], fb[j], acc[i][j]);
    }
    if (s + 1 < nst) {
      store_stage(cur ^ 1);
    }
    __syncthreads();
  }

  // Epilogue: 32x32 accumulator layout -- lane holds column (lane % 32), rows
  // 8*(v/4) + 4*(lane/32) + v%4 for v in [0, 16).
  const int64_t cb = g.c_batch * batch;
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      int64_t col = n0 + wn * WN + j * 32 + (lane & 31);
      if (col >= g.N) continue;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int64_t row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row >= g.M) continue;
        int64_t off = cb + row * g.ldc_m + col * g.ldc_n;
        if constexpr (OUT == 0) {
          ((uint16_t*)g.c)[off] = f32_to_bf16(acc[i][j][v]);
        } else if constexpr (OUT == 1) {
          ((float*)g.c)[off] = acc[i][j][v];
        } else if constexpr (OUT == 2) {
          ((int8_t*)g.c)[off] = (int8_t)acc[i][j][v];
        } else if constexpr (OUT == 4) {
          int32_t a32 = acc[i][j][v];
          ((uint16_t*)g.c)[off] = f32_to_bf16(__fmul_rn(fixedpoint_to_float(a32, 31), g.scale[col]));
          if (g.acc_out) g.acc_out[off] = a32;
        } else {
          ((int32_t*)g.c)[off] = acc[i][j][v];
        }
      }
    }
}

template <bool IS_I8, int OUT>
void gemm_launch(hipStream_t s, const GemmDesc& d, void* c, const void* a, const void* b,
                 const float* scale = nullptr, int32_t* acc_out = nullptr) {
  constexpr int BM = 128, BN = 128;
  GemmArgs g;
  g.a = (const uint8_t*)a;
  g.b = (const uint8_t*)b;
  g.c = c;
  g.M = d.M;
  g.N = d.N;
  g.K = d.K;
  g.lda = d.lda;
  g.ldb = d.ldb;
  g.ldc_m = d.ldc_m;
  g.ldc_n = d.ldc_n;
  g.a_batch = d.a_batch;
  g.b_batch = d.b_batch;
  g.c_batch = d.c_batch;
  g.scale = scale;
  g.acc_out = acc_out;
  g.tiles_m = (int)((d.M + BM - 1) / BM);
  g.tiles_n = (int)((d.N + BN - 1) / BN);
  size_t lds = (size_t)2 * (BM + BN) * kRowB;
  static bool attr_set = false;  // gfx950 LDS is 160 KiB; dynamic LDS above 64 KiB must be opted into
  if (!attr_set) {
    FO_HIP(hipFuncSetAttribute((const void*)k_gemm<IS_I8, OUT, BM, BN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds));
    attr_set = true;
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)d.batch);
  hipLaunchKernelGGL((k_gemm<IS_I8, OUT, BM, BN>), grid, dim3(256), lds, s, g);
  FO_HIP(hipGetLastError());
}

}  // namespace

bool gemm_aligned(const void* a, const void* b, fo_dtype in_t, const GemmDesc& d) {
  int64_t eb = in_t == FO_I8 ? 1 : 2;
  return ((uintptr_t)a % 16) == 0 && ((uintptr_t)b % 16) == 0 && (d.lda * eb) % 16 == 0 && (d.ldb * eb) % 16 == 0 &&
         (d.K * eb) % 16 == 0 && (d.a_batch * eb) % 16 == 0 && (d.b_batch * eb) % 16 == 0 && d.M < (1ll << 31) &&
         d.N < (1ll << 31) && d.batch < 65536;
}

bool gemm_supported(fo_dtype in_t, fo_dtype out_t) {
  return (in_t == FO_BF16 && (out_t == FO_BF16 || out_t == FO_F32)) ||
         (in_t == FO_I8 && (out_t == FO_I8 || out_t == FO_I32));
}

void launch_gemm(hipStream_t s, void* c, const void* a, const void* b, fo_dtype in_t, fo_dtype out_t,
                 const GemmDesc& d) {
  // 16-byte fragment loads need 16-byte aligned rows.
  require(gemm_aligned(a, b, in_t, d), "gemm: operands not 16-byte aligned or shape too large");
  if (in_t == FO_BF16 && out_t == FO_BF16) return gemm_launch<false, 0>(s, d, c, a, b);
  if (in_t == FO_BF16 && out_t == FO_F32) return gemm_launch<false, 1>(s, d, c, a, b);
  if (in_t == FO_I8 && out_t == FO_I8) return gemm_launch<true, 2>(s, d, c, a, b);
  if (in_t == FO_I8 && out_t == FO_I32) return gemm_launch<true, 3>(s, d, c, a, b);
  throw InvalidArg("gemm: unsupported dtype pair");
}

void launch_w8a8(hipStream_t s, uint16_t* out, int32_t* acc_out, const int8_t* a, const int8_t* w, const float* scale,
                 int64_t m, int64_t n, int64_t k) {
  GemmDesc d;
  d.M = m;
  d.N = n;
  d.K = k;
  d.lda = k;
  d.ldb = k;
  d.ldc_m = n;
  d.ldc_n = 1;
  require(gemm_aligned(a, w, FO_I8, d), "w8a8: k must be a multiple of 16 and operands 16-byte aligned");
  gemm_launch<true, 4>(s, d, out, a, w, scale, acc_out);
}

}  // namespace fo
