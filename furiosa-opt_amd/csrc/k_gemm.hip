// MFMA contraction for the tensor-unit path: C[m, n] = sum_k A[m, k] * B[n, k], both operands
// contiguous along k (the K-major layout the mapped GEMM config resolves to: lhs m![M/8, M%8, K],
// rhs m![N, K]). The emulator's fold is BufStorage::contraction_in (storage/buf.rs:401-447):
// widen, accumulate (f32 for bf16, i32 for i8), narrow once per output cell.
//
// Tiling (gfx950, wave64): a block of WM x WN waves owns a BM x BN tile; each wave owns
// (BM/WM) x (BN/WN) as a grid of 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16 /
// v_mfma_i32_32x32x32_i8). K advances 128 bytes per stage. Stages are double-buffered in LDS with
// the next stage's global loads in flight during the current stage's MFMAs, and the LDS fragments
// of the next 32-byte k-step are read while the current k-step's MFMAs issue. LDS rows are padded
// by 16 bytes: a 16-byte fragment read by 32 lanes at stride 144 B covers all 64 banks once per
// 16 lanes. Blocks are ordered XCD-aware so the tiles that share A rows / B columns run on the same
// XCD's L2. Row-major bf16 / i8 results are restaged through LDS and written as 16-byte rows.
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

constexpr int kBKB = 128;         // K bytes per stage
constexpr int kRowB = kBKB + 16;  // padded LDS row stride in bytes

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
  int64_t M, N, K;                 // K in elements
  int64_t lda, ldb, ldc_m, ldc_n;  // elements
  int64_t a_batch, b_batch, c_batch;
  int32_t tiles_m, tiles_n;
  const float* scale;  // OUT == 4: per-column dequant scale
  int32_t* acc_out;    // OUT == 4: optional raw i32 accumulators (row-major, ldc_m / ldc_n)
};

template <int OUT>
struct OutT;
template <>
struct OutT<0> {
  using T = uint16_t;
};
template <>
struct OutT<1> {
  using T = float;
};
template <>
struct OutT<2> {
  using T = int8_t;
};
template <>
struct OutT<3> {
  using T = int32_t;
};
template <>
struct OutT<4> {
  using T = uint16_t;
};

// OUT: 0 = bf16 (from f32), 1 = f32, 2 = i8 (wrap), 3 = i32,
//      4 = W8A8 dequant: bf16(fixedpoint_to_float(acc, 31) * scale[col]) (+ optional raw i32)
template <bool IS_I8, int OUT>
__device__ __forceinline__ typename OutT<OUT>::T convert_out(typename MfmaT<IS_I8>::acc_t const& a, int v, float sc) {
  if constexpr (OUT == 0) {
    return f32_to_bf16(a[v]);
  } else if constexpr (OUT == 1) {
    return a[v];
  } else if constexpr (OUT == 2) {
    return (int8_t)a[v];
  } else if constexpr (OUT == 3) {
    return a[v];
  } else {
    return f32_to_bf16(__fmul_rn(fixedpoint_to_float((int32_t)a[v], 31), sc));
  }
}

template <bool IS_I8, int OUT, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) k_gemm(GemmArgs g) {
  using M = MfmaT<IS_I8>;
  using acc_t = typename M::acc_t;
  using out_t = typename OutT<OUT>::T;
  constexpr int NT = 64 * WM * WN;
  constexpr int EB = IS_I8 ? 1 : 2;  // element bytes
  constexpr int TWM = BM / WM, TWN = BN / WN;  // wave tile
  constexpr int TM = TWM / 32, TN = TWN / 32;
  constexpr int A_LOADS = BM * kBKB / 16 / NT;  // 16-byte loads per thread per stage
  constexpr int B_LOADS = BN * kBKB / 16 / NT;
  static_assert(A_LOADS * NT * 16 == BM * kBKB && B_LOADS * NT * 16 == BN * kBKB, "tile/threads mismatch");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  auto sA = [&](int buf) { return smem + buf * (BM * kRowB); };
  auto sB = [&](int buf) { return smem + 2 * BM * kRowB + buf * (BN * kRowB); };

  // Tile order: consecutive block ids go round-robin over the 8 XCDs; regroup so each XCD walks a
  // contiguous range of tiles, ordered in groups of 8 tile-rows so neighbours share operands in L2.
  const int ntiles = g.tiles_m * g.tiles_n;
  int bid = blockIdx.x;
  int tile = bid;
  if ((ntiles % 8) == 0) tile = (bid % 8) * (ntiles / 8) + bid / 8;
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
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t KB = g.K * EB;  // K in bytes

  const uint8_t* A = g.a + (g.a_batch * batch) * EB;
  const uint8_t* B = g.b + (g.b_batch * batch) * EB;

  // Global load assignment: chunk c = tid + i*NT is row c/8, byte column (c%8)*16. Interior tiles
  // (the whole BM x BN block in range and K a whole number of stages) load without bounds checks;
  // the test is uniform over the block, so edge tiles take the checked path without divergence.
  const bool interior = (m0 + BM <= g.M) && (n0 + BN <= g.N) && (KB % kBKB == 0);
  i32x4_t ra[A_LOADS], rb[B_LOADS];
  const uint8_t* a_base[A_LOADS];
  const uint8_t* b_base[B_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; ++i) {
    int c = tid + i * NT;
    a_base[i] = A + ((m0 + (c >> 3)) * g.lda) * EB + (c & 7) * 16;
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; ++i) {
    int c = tid + i * NT;
    b_base[i] = B + ((n0 + (c >> 3)) * g.ldb) * EB + (c & 7) * 16;
  }
  auto load_stage = [&](int64_t kb) {
    if (interior) {
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) ra[i] = *(const i32x4_t*)(a_base[i] + kb);
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) rb[i] = *(const i32x4_t*)(b_base[i] + kb);
    } else {
#pragma unroll
      for (int i = 0; i < A_LOADS; ++i) {
        int c = tid + i * NT;
        bool ok = (m0 + (c >> 3) < g.M) && (kb + (c & 7) * 16 < KB);
        ra[i] = ok ? *(const i32x4_t*)(a_base[i] + kb) : i32x4_t{0, 0, 0, 0};
      }
#pragma unroll
      for (int i = 0; i < B_LOADS; ++i) {
        int c = tid + i * NT;
        bool ok = (n0 + (c >> 3) < g.N) && (kb + (c & 7) * 16 < KB);
        rb[i] = ok ? *(const i32x4_t*)(b_base[i] + kb) : i32x4_t{0, 0, 0, 0};
      }
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int c = tid + i * NT;
      *(i32x4_t*)(sA(buf) + (c >> 3) * kRowB + (c & 7) * 16) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      int c = tid + i * NT;
      *(i32x4_t*)(sB(buf) + (c >> 3) * kRowB + (c & 7) * 16) = rb[i];
    }
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  const int frow = lane & 31;         // fragment row within a 32-row tile
  const int fcol = (lane >> 5) * 16;  // this lane's 16 bytes within a 32-byte k-step
  const int arow0 = wm * TWM + frow, brow0 = wn * TWN + frow;

  // Pipeline: at the top of iteration s, LDS buffer (s & 1) holds stage s and the registers hold
  // stage s + 1. The iteration reads its first fragments, writes stage s + 1 into the other buffer
  // (last read in iteration s - 1, fenced by that iteration's barrier), issues the global loads of
  // stage s + 2, and runs stage s's MFMAs with the next k-step's fragments read ahead.
  const int nst = (int)((KB + kBKB - 1) / kBKB);
  load_stage(0);
  store_stage(0);
  if (nst > 1) load_stage(kBKB);
  __syncthreads();

  for (int s = 0; s < nst; ++s) {
    const int cur = s & 1;
    const uint8_t* a_s = sA(cur);
    const uint8_t* b_s = sB(cur);
    i32x4_t fa[2][TM], fb[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[0][i] = *(const i32x4_t*)(a_s + (arow0 + i * 32) * kRowB + fcol);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[0][j] = *(const i32x4_t*)(b_s + (brow0 + j * 32) * kRowB + fcol);
    if (s + 1 < nst) {
      store_stage(cur ^ 1);
      if (s + 2 < nst) load_stage((int64_t)(s + 2) * kBKB);
    }
#pragma unroll
    for (int kk = 0; kk < kBKB / 32; ++kk) {
      const int p = kk & 1;
      if (kk + 1 < kBKB / 32) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
          fa[p ^ 1][i] = *(const i32x4_t*)(a_s + (arow0 + i * 32) * kRowB + (kk + 1) * 32 + fcol);
#pragma unroll
        for (int j = 0; j < TN; ++j)
          fb[p ^ 1][j] = *(const i32x4_t*)(b_s + (brow0 + j * 32) * kRowB + (kk + 1) * 32 + fcol);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(fa[p][i], fb[p][j], acc[i][j]);
    }
    __syncthreads();
  }

  // Epilogue. Accumulator layout of a 32x32 tile: lane holds column (lane % 32), rows
  // 8*(v/4) + 4*(lane/32) + v%4 for v in [0, 16).
  const int64_t cb = g.c_batch * batch;
  const bool full_tile = (m0 + BM <= g.M) && (n0 + BN <= g.N);
  constexpr int OB = (int)sizeof(out_t);
  constexpr int CROW = BN * OB + 16;  // padded LDS row of the staged C tile
  if (OUT != 4 && full_tile && g.ldc_n == 1 && (g.ldc_m * OB) % 16 == 0 && (g.c_batch * OB) % 16 == 0 &&
      BM * CROW <= 2 * (BM + BN) * kRowB && ((uintptr_t)g.c % 16) == 0) {
    // Stage the tile in LDS, then write 16-byte rows.
    uint8_t* sc = smem;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        int col = wn * TWN + j * 32 + (lane & 31);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          int row = wm * TWM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
          *(out_t*)(sc + row * CROW + col * OB) = convert_out<IS_I8, OUT>(acc[i][j], v, 0.f);
        }
      }
    __syncthreads();
    constexpr int CHUNKS = BM * BN * OB / 16;
    constexpr int ROWCH = BN * OB / 16;
    out_t* C = (out_t*)g.c;
    for (int c = tid; c < CHUNKS; c += NT) {
      int row = c / ROWCH, ch = c % ROWCH;
      i32x4_t val = *(const i32x4_t*)(sc + row * CROW + ch * 16);
      *(i32x4_t*)((uint8_t*)(C + cb + (m0 + row) * g.ldc_m + n0) + ch * 16) = val;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      int64_t col = n0 + wn * TWN + j * 32 + (lane & 31);
      if (col >= g.N) continue;
      float sc = 0.f;
      if constexpr (OUT == 4) sc = g.scale[col];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        int64_t row = m0 + wm * TWM + i * 32 + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row >= g.M) continue;
        int64_t off = cb + row * g.ldc_m + col * g.ldc_n;
        ((out_t*)g.c)[off] = convert_out<IS_I8, OUT>(acc[i][j], v, sc);
        if constexpr (OUT == 4) {
          if (g.acc_out) g.acc_out[off] = (int32_t)acc[i][j][v];
        }
      }
    }
}

template <bool IS_I8, int OUT, int BM, int BN, int WM, int WN>
void gemm_launch_cfg(hipStream_t s, const GemmDesc& d, void* c, const void* a, const void* b, const float* scale,
                     int32_t* acc_out) {
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
    FO_HIP(hipFuncSetAttribute((const void*)k_gemm<IS_I8, OUT, BM, BN, WM, WN>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set = true;
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)d.batch);
  hipLaunchKernelGGL((k_gemm<IS_I8, OUT, BM, BN, WM, WN>), grid, dim3(64 * WM * WN), lds, s, g);
  FO_HIP(hipGetLastError());
}

// Tile choice: 256x256 with 8 waves (one tile per CU at 4096^2) when the problem is large,
// 128x128 otherwise (measured best on MI355X among 128, 256/4-wave and 256/8-wave).
// FO_GEMM_TILE overrides it for measurement: 128, 256 (4 waves of 128x128) or 2568 (8 waves).
template <bool IS_I8, int OUT>
void gemm_launch(hipStream_t s, const GemmDesc& d, void* c, const void* a, const void* b,
                 const float* scale = nullptr, int32_t* acc_out = nullptr) {
  static int forced = [] {
    const char* e = getenv("FO_GEMM_TILE");
    return e ? atoi(e) : 0;
  }();
  int64_t tiles256 = ((d.M + 255) / 256) * ((d.N + 255) / 256) * d.batch;
  int choice = forced ? forced : (tiles256 >= 128 ? 2568 : 128);
  if (choice == 2568) return gemm_launch_cfg<IS_I8, OUT, 256, 256, 2, 4>(s, d, c, a, b, scale, acc_out);
  if (choice == 256) return gemm_launch_cfg<IS_I8, OUT, 256, 256, 2, 2>(s, d, c, a, b, scale, acc_out);
  return gemm_launch_cfg<IS_I8, OUT, 128, 128, 2, 2>(s, d, c, a, b, scale, acc_out);
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
