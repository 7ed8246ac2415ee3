// MFMA contraction for the tensor-unit path: C[m, n] = sum_k A[m, k] * B[n, k], both operands
// contiguous along k (the K-major layout the mapped GEMM config resolves to: lhs m![M/8, M%8, K],
// rhs m![N, K]). The emulator's fold is BufStorage::contraction_in (storage/buf.rs:401-447):
// widen, accumulate (f32 for bf16, i32 for i8), narrow once per output cell.
//
// Tiling (gfx950, wave64): a block of WM x WN waves owns a BM x BN tile; each wave owns
// (BM/WM) x (BN/WN) as a grid of 32x32 MFMA tiles (v_mfma_f32_32x32x16_bf16 /
// v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x64_f8f6f4 for the two 8-bit float formats, OCP E4M3
// and E5M2, the encodings of f8e4m3 / f8e5m2). K advances kRB bytes per stage; kNS stages rotate
// through LDS. The
// DMA refilling a buffer is issued right after the barrier that releases it, and each stage waits
// only for its own DMA (vmcnt counts the younger ones).
//
// Operand staging: global -> LDS by buffer_load_dwordx4 ... lds (LDS DMA: each lane's 16 bytes
// land at the wave's LDS base + 16 * lane, no VGPR round trip and no ds_write). A wave's
// 1 KiB DMA covers 8 rows of 128 bytes; the lane -> (row, chunk) assignment stores chunk c of row
// r at slot c ^ ((r >> 1) & 7), so the 16 lanes of one 16-byte fragment read (16 consecutive rows,
// one chunk) touch 16 distinct 16-byte bank groups. Rows past the operand's extent read as zero
// (buffer range check); chunks past K are pointed outside the range for the same effect.
//
// Epilogue: the MFMA operands are swapped (B fragments as the A operand) so each lane holds four
// consecutive output columns of one row, stored directly to global memory.
//
// Within one MFMA the hardware's k order is irrelevant: A and B fragments are loaded with the same
// k -> (lane, element) map, and the sum over k is order-free up to f32 rounding (exact for i32).
#include <hip/hip_runtime.h>

#include <type_traits>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16_t;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2_t;
typedef __attribute__((__vector_size__(8 * sizeof(int)))) int i32x8_t;

constexpr int kRB = 128;  // K bytes per row per stage (four 32-byte MFMA k-steps)
constexpr int kNS = 2;    // LDS stages (double buffer; 64-byte stages x4 measured slower: more barriers)
constexpr int kCPR = kRB / 16;                  // 16-byte chunks per row
constexpr int kRPC = 1024 / kRB;                // rows per 1 KiB wave DMA
constexpr int kSwzShift = kRB == 64 ? 2 : 1;    // rows sharing a bank-group offset: 16 / kCPR

// s_waitcnt immediate (gfx9 encoding): vector memory count <= n, LDS/scalar count 0, export any.
constexpr int waitcnt_vm_lgkm0(int n) { return (n & 15) | (7 << 4) | ((n >> 4) << 14); }

// Operand kinds. Per MFMA, each lane supplies FRAG bytes of k (16 for bf16 / i8, 32 for the
// 8-bit floats: k = 64 per instruction); KSTEP = 2 * FRAG bytes of k per row per MFMA.
enum Kind { kBf16 = 0, kI8 = 1, kF8E4M3 = 2, kF8E5M2 = 3 };

template <int KIND>
struct MfmaT;
template <>
struct MfmaT<kBf16> {
  using acc_t = f32x16_t;
  using frag_t = i32x4_t;
  static constexpr int EB = 2;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                   0, 0, 0);
  }
};
template <>
struct MfmaT<kI8> {
  using acc_t = i32x16_t;
  using frag_t = i32x4_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
// The f8f6f4 instruction with both operand formats set (cbsz / blgp: 0 = E4M3, 1 = E5M2) and no
// block scale. It sums a 64-wide k block at reduced internal precision: measured on MI355X, the
// error of one instruction is about 2e-5 of sum |a_k b_k| on average, 1.6e-4 at most (an f32
// sequential fold: 3e-7), the products themselves being exact.
template <>
struct MfmaT<kF8E4M3> {
  using acc_t = f32x16_t;
  using frag_t = i32x8_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
};
template <>
struct MfmaT<kF8E5M2> {
  using acc_t = f32x16_t;
  using frag_t = i32x8_t;
  static constexpr int EB = 1;
  static __device__ __forceinline__ acc_t mma(const frag_t& a, const frag_t& b, const acc_t& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 1, 0, 0, 0, 0);
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
template <>
struct OutT<5> {
  using T = uint8_t;
};
template <>
struct OutT<6> {
  using T = uint8_t;
};

// OUT: 0 = bf16 (from f32), 1 = f32, 2 = i8 (wrap), 3 = i32,
//      4 = W8A8 dequant: bf16(fixedpoint_to_float(acc, 31) * scale[col]) (+ optional raw i32),
//      5 = f8e4m3 (from f32), 6 = f8e5m2 (from f32)
template <int KIND, int OUT>
__device__ __forceinline__ typename OutT<OUT>::T convert_out(typename MfmaT<KIND>::acc_t const& a, int v, float sc) {
  if constexpr (OUT == 5) {
    return f32_to_f8e4m3(a[v]);
  } else if constexpr (OUT == 6) {
    return f32_to_f8e5m2(a[v]);
  } else if constexpr (OUT == 0) {
    return f32_to_bf16(a[v]);
  } else if constexpr (OUT == 1) {
    return a[v];
  } else if constexpr (OUT == 2) {
    return (int8_t)a[v];
  } else if constexpr (OUT == 3) {
    return a[v];
  } else {
    // fixedpoint_to_float(acc, 31) is the nearest f32 of acc: the i32 -> f32 conversion (RNE)
    return f32_to_bf16(__fmul_rn((float)(int32_t)a[v], sc));
  }
}

// LDS address space pointer for the DMA builtin.
typedef __attribute__((address_space(3))) void* lds_ptr_t;

// Values the compiler cannot prove wave-uniform (it otherwise builds the buffer descriptor in
// VGPRs and wraps every DMA in a readfirstlane loop); they are uniform by construction.
__device__ __forceinline__ void* uniform_ptr(const void* p) {
  uint64_t v = (uint64_t)p;
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (void*)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ int uniform_i32(int64_t v) { return __builtin_amdgcn_readfirstlane((int)v); }

// Two 4-column groups of 16-bit outputs (vg and vg + 1 of an MFMA tile: lanes l < 32 hold columns
// 8 vg + 0..3 of row l, lanes l + 32 columns 8 vg + 4..7) regrouped across the wave halves by
// v_permlane32_swap: lane l < 32 gets columns 8 vg + 0..7 of row l, lane l + 32 columns
// 8 (vg + 1) + 0..7, so each lane stores 16 contiguous bytes.
// The same regrouping for 8-bit outputs: 4 columns are one dword, 8 columns 8 bytes.
__device__ __forceinline__ i32x2_t regroup8_b(uint32_t a, uint32_t b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  return i32x2_t{(int)r[0], (int)r[1]};
}
__device__ __forceinline__ i32x4_t regroup8(i32x2_t a, i32x2_t b) {
  const auto r0 = __builtin_amdgcn_permlane32_swap((uint32_t)a[0], (uint32_t)b[0], false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap((uint32_t)a[1], (uint32_t)b[1], false, false);
  return i32x4_t{(int)r0[0], (int)r1[0], (int)r0[1], (int)r1[1]};
}

template <int KIND, int OUT, int BM, int BN, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN) k_gemm(GemmArgs g) {
  using M = MfmaT<KIND>;
  using acc_t = typename M::acc_t;
  using frag_t = typename M::frag_t;
  using out_t = typename OutT<OUT>::T;
  constexpr int W = WM * WN;
  constexpr int EB = M::EB;                    // element bytes
  constexpr int FRAG = (int)sizeof(frag_t);    // k bytes per lane per MFMA
  constexpr int KSTEP = 2 * FRAG;              // k bytes per row per MFMA
  constexpr int TWM = BM / WM, TWN = BN / WN;  // wave tile
  constexpr int TM = TWM / 32, TN = TWN / 32;
  constexpr int A_CH = BM / kRPC / W;  // 1 KiB DMA chunks of A per wave per stage
  constexpr int B_CH = BN / kRPC / W;
  static_assert(A_CH * kRPC * W == BM && B_CH * kRPC * W == BN, "tile/waves mismatch");
  constexpr int PER = A_CH + B_CH;  // DMA instructions per wave per stage
  constexpr int STAGE = (BM + BN) * kRB;

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  auto sA = [&](int buf) { return smem + buf * STAGE; };
  auto sB = [&](int buf) { return smem + buf * STAGE + BM * kRB; };

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
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const uint32_t KB = (uint32_t)(g.K * EB);  // K in bytes

  // Buffer resources based at the tile's first row, extent = the bytes its valid rows span.
  const int64_t rows_a = min((int64_t)BM, g.M - m0), rows_b = min((int64_t)BN, g.N - n0);
  const uint8_t* Abase = g.a + (g.a_batch * batch + m0 * g.lda) * EB;
  const uint8_t* Bbase = g.b + (g.b_batch * batch + n0 * g.ldb) * EB;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(Abase), (short)0, uniform_i32((rows_a - 1) * g.lda * EB + KB), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(Bbase), (short)0, uniform_i32((rows_b - 1) * g.ldb * EB + KB), 0x00020000);

  // DMA source offsets: lane l of chunk q fills LDS slot l % kCPR of tile row r = kRPC q + l / kCPR
  // with global chunk (l % kCPR) ^ swz(r), swz(r) = (r >> kSwzShift) & (kCPR - 1).
  uint32_t a_off[A_CH], a_kc[A_CH], b_off[B_CH], b_kc[B_CH];
#pragma unroll
  for (int i = 0; i < A_CH; ++i) {
    int r = kRPC * (wave * A_CH + i) + lane / kCPR;
    int c = (lane % kCPR) ^ ((r >> kSwzShift) & (kCPR - 1));
    a_kc[i] = (uint32_t)c * 16;
    a_off[i] = (uint32_t)(r * g.lda * EB) + a_kc[i];
  }
#pragma unroll
  for (int i = 0; i < B_CH; ++i) {
    int r = kRPC * (wave * B_CH + i) + lane / kCPR;
    int c = (lane % kCPR) ^ ((r >> kSwzShift) & (kCPR - 1));
    b_kc[i] = (uint32_t)c * 16;
    b_off[i] = (uint32_t)(r * g.ldb * EB) + b_kc[i];
  }
  // DMA instructions [lo, hi) of stage st (A chunks first, then B). A FULL stage lies within K:
  // the stage offset goes in the scalar offset and no lane needs a check. Otherwise (the last
  // stage may be partial) chunks past K get an out-of-range offset and read zero. FULL is a
  // constant at every (inlined) call.
  auto issue_rng = [&](int st, int lo, int hi, bool FULL) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass drops the kernel stubs over these builtins
    const uint32_t kb = (uint32_t)st * kRB;
    const int buf = st % kNS;
    const bool tail = !FULL && kb + kRB > KB;  // uniform
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      if (i < lo || i >= hi) continue;
      if (FULL) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(sA(buf) + (wave * A_CH + i) * 1024), 16, a_off[i], kb, 0,
                                                 0);
      } else {
        uint32_t off = a_off[i] + kb;
        if (tail && kb + a_kc[i] >= KB) off = 0x80000000u;  // past K: out of range, reads zero
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(sA(buf) + (wave * A_CH + i) * 1024), 16, off, 0, 0, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      if (A_CH + i < lo || A_CH + i >= hi) continue;
      if (FULL) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(sB(buf) + (wave * B_CH + i) * 1024), 16, b_off[i], kb, 0,
                                                 0);
      } else {
        uint32_t off = b_off[i] + kb;
        if (tail && kb + b_kc[i] >= KB) off = 0x80000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(sB(buf) + (wave * B_CH + i) * 1024), 16, off, 0, 0, 0);
      }
    }
#endif
  };

  acc_t acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0;

  // Fragment reads: lane (frow, half) takes FRAG bytes of k-step kk: the 16-byte chunks
  // (KSTEP / 16) kk + (FRAG / 16) half + e of row frow (+ 32i), found at slot chunk ^ swz; rows of
  // a fragment tile start at multiples of 32, so swz depends on frow only.
  const int frow = lane & 31, half = lane >> 5;
  const int swz = (frow >> kSwzShift) & (kCPR - 1);
  const int a_row = (wm * TWM + frow) * kRB, b_row = (wn * TWN + frow) * kRB;
  auto slot = [&](int kk, int e) { return (((KSTEP / 16) * kk + (FRAG / 16) * half + e) ^ swz) * 16; };

  const int nst = (int)((KB + kRB - 1) / kRB);
  constexpr int KST = kRB / KSTEP;  // MFMA k-steps per stage
  static_assert(KST % 2 == 0, "fragment double-buffer parity assumes an even k-step count");
  // Stage s's DMA is complete once at most the younger stages' DMAs are outstanding; after the
  // barrier every wave's is, and every wave has its fragments of the previous stage in registers,
  // so that stage's buffer can be refilled. The barrier carries no memory fence (that would drain
  // every DMA); the compiler barriers keep LDS accesses on their side of it.
  auto stage_ready = [&](int s) {
    // DMAs in flight younger than stage s: the prologue fills all kNS buffers; afterwards the
    // refill of stage s - 1's buffer (stage s - 1 + kNS) is issued after this barrier.
    const int ahead = min(nst - 1 - s, s == 0 ? kNS - 1 : kNS - 2);
    if (ahead >= 3)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(3 * PER));
    else if (ahead == 2)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * PER));
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(PER));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
  };
  frag_t fa[2][TM], fb[2][TN];
  auto read_frags = [&](int buf, int kk, int p) {
    const uint8_t* a_s = sA(buf);
    const uint8_t* b_s = sB(buf);
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const uint8_t* r = a_s + a_row + i * 32 * kRB;
#pragma unroll
      for (int e = 0; e < FRAG / 16; ++e) {
        i32x4_t q = *(const i32x4_t*)(r + slot(kk, e));
#pragma unroll
        for (int w = 0; w < 4; ++w) fa[p][i][4 * e + w] = q[w];
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const uint8_t* r = b_s + b_row + j * 32 * kRB;
#pragma unroll
      for (int e = 0; e < FRAG / 16; ++e) {
        i32x4_t q = *(const i32x4_t*)(r + slot(kk, e));
#pragma unroll
        for (int w = 0; w < 4; ++w) fb[p][j][4 * e + w] = q[w];
      }
    }
  };

#pragma unroll
  for (int st = 0; st < kNS; ++st)
    if (st < nst) issue_rng(st, 0, PER, false);
  stage_ready(0);
  read_frags(0, 0, 0);
  // Pipeline over the flattened k-steps t = s * KST + kk: the fragments of t + 1 are read while
  // t's MFMAs issue. Crossing into stage s + 1, its readiness barrier comes after the last
  // fragments of stage s were read and before t's MFMAs, which then cover the latency of the
  // first reads from stage s + 1.
  // The refill of the buffer freed by that barrier is issued in NP parts: the first after t's
  // MFMAs, the others after the next k-steps' fragment reads. A CU takes in about 64 B of DMA per
  // clock, so one burst of a whole stage (64 KiB) right after the barrier held every wave at its
  // DMA issue, with its MFMAs queued behind, for ~1000 of the ~3600 clocks of a stage (per-stage
  // timestamps); split and placed this way the bf16 GEMM runs 9-10% faster. The scheduling
  // barriers keep the MFMAs on their side of the readiness barrier and of the first part.
  // Two k-steps per stage (the 8-bit floats): one part after the MFMAs measured 3-4% faster.
  constexpr int NP = KST <= 2 ? 1 : 2;
  // S (a constant at each inlined call): s >= 1 and every stage refilled here is full.
  auto stage = [&](int s, bool S) __attribute__((always_inline)) {
#pragma unroll
    for (int kk = 0; kk < KST; ++kk) {
      const int p = kk & 1;  // KST is even: the fragment buffer parity restarts each stage
      if (kk + 1 < KST) {
        read_frags(s % kNS, kk + 1, p ^ 1);
        const int r = s + kNS - 1;  // refilled after stage s - 1's last barrier
        if (kk + 1 < NP && (S || (r >= kNS && r < nst)))
          issue_rng(r, (kk + 1) * PER / NP, (kk + 2) * PER / NP, S);
      } else if (S || s + 1 < nst) {
        __builtin_amdgcn_sched_barrier(0);
        stage_ready(s + 1);
        __builtin_amdgcn_sched_barrier(0);
        read_frags((s + 1) % kNS, 0, p ^ 1);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = M::mma(fb[p][j], fa[p][i], acc[i][j]);
      __builtin_amdgcn_iglp_opt(0);  // interleave the fragment reads with the MFMAs
      if (kk + 1 == KST && (S || s + kNS < nst)) {
        __builtin_amdgcn_sched_barrier(0);
        issue_rng(s + kNS, 0, PER / NP, S);
      }
    }
  };
  // Steady stages: s >= 1 (the prologue issued stages 0 .. kNS - 1) and s + kNS <= nst - 2 (every
  // stage they refill lies before the last, the only one that may be partial).
  int s = 0;
  if (nst > 0) stage(s++, false);
  for (; s + kNS + 2 <= nst; ++s) stage(s, true);
  for (; s < nst; ++s) stage(s, false);

  // Epilogue. With B as the MFMA's A operand, lane holds row m = 32i + (lane % 32) of the wave
  // tile and columns n = 32j + 8*(v/4) + 4*(lane/32) + v%4: four consecutive columns per v / 4.
  const int64_t cb = g.c_batch * batch;
  out_t* C = (out_t*)g.c;
  constexpr int OB = (int)sizeof(out_t);
  const bool vec = g.ldc_n == 1 && (g.ldc_m * OB) % (4 * OB) == 0 && (cb * OB) % (4 * OB) == 0 &&
                   ((uintptr_t)g.c % (4 * OB)) == 0 && (OUT != 4 || ((uintptr_t)g.scale % 16) == 0);
  if constexpr (OB == 1) {
    // 8-bit outputs of a wave tile wholly inside C: 8-byte stores of 8 columns.
    const bool wide = vec && g.ldc_m % 8 == 0 && cb % 8 == 0 && ((uintptr_t)g.c % 8) == 0 &&
                      m0 + wm * TWM + TWM <= g.M && n0 + wn * TWN + TWN <= g.N;
    if (wide) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t row = m0 + wm * TWM + i * 32 + frow;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int vp = 0; vp < 4; vp += 2) {
            uint32_t w[2];
#pragma unroll
            for (int d = 0; d < 2; ++d) {
              out_t o4[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) o4[e] = convert_out<KIND, OUT>(acc[i][j], (vp + d) * 4 + e, 0.f);
              w[d] = __builtin_bit_cast(uint32_t, o4);
            }
            const int64_t col = n0 + wn * TWN + j * 32 + 8 * vp + 8 * half;
            *(i32x2_t*)(C + cb + row * g.ldc_m + col) = regroup8_b(w[0], w[1]);
          }
      }
      return;
    }
  }
  if constexpr (OB == 2) {
    // 16-bit outputs of a wave tile wholly inside C: 16-byte stores of 8 columns (two per row
    // and instruction) instead of 8-byte ones.
    const bool wide = vec && g.ldc_m % 8 == 0 && cb % 8 == 0 && ((uintptr_t)g.c % 16) == 0 &&
                      (OUT != 4 || !g.acc_out) && m0 + wm * TWM + TWM <= g.M && n0 + wn * TWN + TWN <= g.N;
    if (wide) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t row = m0 + wm * TWM + i * 32 + frow;
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int vp = 0; vp < 4; vp += 2) {
            i32x2_t w[2];
#pragma unroll
            for (int d = 0; d < 2; ++d) {
              const int vg = vp + d;
              float sc[4] = {0.f, 0.f, 0.f, 0.f};
              if constexpr (OUT == 4) {
                typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
                f32x4_t s4 = *(const f32x4_t*)(g.scale + n0 + wn * TWN + j * 32 + 8 * vg + 4 * half);
#pragma unroll
                for (int e = 0; e < 4; ++e) sc[e] = s4[e];
              }
              out_t o4[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) o4[e] = convert_out<KIND, OUT>(acc[i][j], vg * 4 + e, sc[e]);
              w[d] = __builtin_bit_cast(i32x2_t, o4);
            }
            const int64_t col = n0 + wn * TWN + j * 32 + 8 * vp + 8 * half;
            *(i32x4_t*)(C + cb + row * g.ldc_m + col) = regroup8(w[0], w[1]);
          }
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t row = m0 + wm * TWM + i * 32 + frow;
    if (row >= g.M) continue;
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        const int64_t col = n0 + wn * TWN + j * 32 + 8 * vg + 4 * half;
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        if (vec && col + 3 < g.N) {
          if constexpr (OUT == 4) {
            typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
            f32x4_t s4 = *(const f32x4_t*)(g.scale + col);
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[e] = s4[e];
          }
          out_t o4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = convert_out<KIND, OUT>(acc[i][j], vg * 4 + e, sc[e]);
          int64_t off = cb + row * g.ldc_m + col;
          if constexpr (OB == 1) {
            *(uint32_t*)(C + off) = __builtin_bit_cast(uint32_t, o4);
          } else if constexpr (OB == 2) {
            *(i32x2_t*)(C + off) = __builtin_bit_cast(i32x2_t, o4);
          } else {
            *(i32x4_t*)(C + off) = __builtin_bit_cast(i32x4_t, o4);
          }
          if constexpr (OUT == 4) {
            if (g.acc_out) {
              i32x4_t a4;
#pragma unroll
              for (int e = 0; e < 4; ++e) a4[e] = (int32_t)acc[i][j][vg * 4 + e];
              *(i32x4_t*)(g.acc_out + off) = a4;
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e >= g.N) continue;
            if constexpr (OUT == 4) sc[e] = g.scale[col + e];
            int64_t off = cb + row * g.ldc_m + (col + e) * g.ldc_n;
            C[off] = convert_out<KIND, OUT>(acc[i][j], vg * 4 + e, sc[e]);
            if constexpr (OUT == 4) {
              if (g.acc_out) g.acc_out[off] = (int32_t)acc[i][j][vg * 4 + e];
            }
          }
        }
      }
  }
}

// ---- four waves of 128x128 (16x16 MFMA tiles) ---------------------------------------------------
//
// The same contraction with one wave per SIMD: a 256x256 block tile split into 2x2 wave tiles of
// 128x128, each an 8x8 grid of 16x16 MFMA tiles (v_mfma_f32_16x16x32_bf16 / v_mfma_i32_16x16x64_i8:
// per instruction each lane supplies 16 bytes of one row -- row lane % 16, bytes 16 (lane / 16) ..
// + 15 of a 64-byte k window). The 256 accumulators per lane live in the accumulation registers,
// the fragments of two k-steps in the vector registers. Per k-step a wave reads 16 fragments for
// 64 MFMAs, a third less LDS traffic per MFMA than the eight-wave form's 128x64 tiles. 128-byte
// stages of k are double-buffered in LDS (the same LDS-DMA staging and XOR swizzle as k_gemm);
// within a k-step, each group of four MFMAs is preceded by one fragment read of the next k-step
// and, after a stage's readiness barrier, one refill DMA instruction, since no second wave on the
// SIMD covers their issue. On MI355X at 4096^3 bf16 this measured 1300-1380 TFLOP/s against
// 1240-1304 for the eight-wave form on the same boxes.
//
// The MFMAs are written as inline assembly with the accumulator tied to the output ("+a"): with
// all 256 accumulation registers holding accumulators, the builtin's untied form made the register
// allocator rotate accumulators through spare registers (~600 copies per 128 MFMAs). As volatile
// statements they also keep their source order with the fragment reads and DMA between them, which
// is the interleave wanted (the scheduler cannot classify them as MFMAs). Since the compiler does not
// see them as MFMAs, the epilogue pads their latency before it reads the accumulators.
template <int KIND>
struct Mfma16;
template <>
struct Mfma16<kBf16> {
  using acc_t = f32x4_t;
  static __device__ __forceinline__ void mma(acc_t& c, const i32x4_t& a, const i32x4_t& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};
template <>
struct Mfma16<kI8> {
  using acc_t = i32x4_t;
  static __device__ __forceinline__ void mma(acc_t& c, const i32x4_t& a, const i32x4_t& b) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
};

// f(std::integral_constant<int, B>{}) ... f(std::integral_constant<int, E - 1>{}): loop indices that
// are compile-time constants however large the body (register arrays stay registers).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int OUT, typename A>
__device__ __forceinline__ typename OutT<OUT>::T cvt4(const A& a, int v, float sc) {
  if constexpr (OUT == 0) {
    return f32_to_bf16(a[v]);
  } else if constexpr (OUT == 1) {
    return a[v];
  } else if constexpr (OUT == 2) {
    return (int8_t)a[v];
  } else if constexpr (OUT == 3) {
    return a[v];
  } else {
    static_assert(OUT == 4, "16x16 tiles: bf16, f32, i8, i32 or the W8A8 dequant");
    // fixedpoint_to_float(acc, 31) is the nearest f32 of acc: the i32 -> f32 conversion (RNE)
    return f32_to_bf16(__fmul_rn((float)(int32_t)a[v], sc));
  }
}

// Elements e and e + 1 of a tile's accumulators as a packed bf16 pair (OUT 0: the f32 sums; OUT 4:
// the W8A8 dequant), by the reference's narrow.
template <int OUT, typename A>
__device__ __forceinline__ uint32_t cvt_pair16(const A& a, int e, float s0, float s1) {
  static_assert(OUT == 0 || OUT == 4, "bf16 outputs");
  if constexpr (OUT == 4)
    return pack_bf16_rule(__fmul_rn((float)(int32_t)a[e], s0), __fmul_rn((float)(int32_t)a[e + 1], s1));
  else
    return pack_bf16_rule(a[e], a[e + 1]);
}

template <int KIND, int OUT, int NSA>
__global__ void __launch_bounds__(256, 1) k_gemm4(GemmArgs g) {
  using MM = Mfma16<KIND>;
  using acc_t = typename MM::acc_t;
  using out_t = typename OutT<OUT>::T;
  constexpr int EB = KIND == kBf16 ? 2 : 1;
  constexpr int BM = 256, BN = 256, W = 4, TT = 8;  // TT x TT MFMA tiles of 16x16 per wave
  constexpr int BKB = 128;                           // bytes of k per row per stage
  constexpr int CPR = BKB / 16;                      // 16-byte chunks per row per stage
  constexpr int RPC = 1024 / BKB;                    // rows per 1 KiB wave DMA
  constexpr int A_CH = BM / RPC / W, B_CH = BN / RPC / W;  // DMA instructions per wave per stage
  constexpr int KST = BKB / 64;                      // MFMA k-steps per stage (64 bytes of k each)
  constexpr int NSB = 2;                             // B buffers; A has NSA
  constexpr int ABYTES = BM * BKB, BBYTES = BN * BKB;
  static_assert(NSA >= NSB && NSA * ABYTES + NSB * BBYTES <= 160 * 1024, "LDS");
  static_assert(A_CH == 8 && B_CH == 8, "one DMA instruction per MFMA group");

  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  auto sA = [&](int buf) { return smem + buf * ABYTES; };
  auto sB = [&](int buf) { return smem + NSA * ABYTES + buf * BBYTES; };

  const int ntiles = g.tiles_m * g.tiles_n;
  int tile = blockIdx.x;
  if ((ntiles % 8) == 0) tile = (tile % 8) * (ntiles / 8) + tile / 8;
  // Each XCD's 32 consecutive tiles form a 4 x 8 block at 4096^2 (4 A and 8 B panels into its L2;
  // 97.96-98.24 against 98.8-99.2 us for the 8 x 4 block of group 8 on one box).
  const int group = 4;
  const int gsize = group * g.tiles_n;
  const int first_m = (tile / gsize) * group;
  const int gm = min(g.tiles_m - first_m, group);
  const int tm = first_m + (tile % gsize) % gm;
  const int tn = (tile % gsize) / gm;
  const int batch = blockIdx.y;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const uint32_t KB = (uint32_t)(g.K * EB);

  const int64_t rows_a = min((int64_t)BM, g.M - m0), rows_b = min((int64_t)BN, g.N - n0);
  const uint8_t* Abase = g.a + (g.a_batch * batch + m0 * g.lda) * EB;
  const uint8_t* Bbase = g.b + (g.b_batch * batch + n0 * g.ldb) * EB;
  const __amdgpu_buffer_rsrc_t ra =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(Abase), (short)0, uniform_i32((rows_a - 1) * g.lda * EB + KB), 0x00020000);
  const __amdgpu_buffer_rsrc_t rb =
      __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(Bbase), (short)0, uniform_i32((rows_b - 1) * g.ldb * EB + KB), 0x00020000);

  // DMA: lane l of chunk q fills LDS slot l % CPR of row r = RPC q + l / CPR with global chunk
  // (l % CPR) ^ swz(r), swz(r) = (r >> 1) & (CPR - 1). Chunks q and q + 2 differ by 2 RPC rows,
  // which leaves swz unchanged, so two per-lane offsets serve every chunk (the rest is a uniform
  // row stride in the scalar offset).
  uint32_t a_off[2], a_kc[2], b_off[2], b_kc[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ra_ = RPC * (wave * A_CH + i) + lane / CPR, rb_ = RPC * (wave * B_CH + i) + lane / CPR;
    a_kc[i] = (uint32_t)(((lane % CPR) ^ ((ra_ >> 1) & (CPR - 1))) * 16);
    a_off[i] = (uint32_t)(ra_ * g.lda * EB) + a_kc[i];
    b_kc[i] = (uint32_t)(((lane % CPR) ^ ((rb_ >> 1) & (CPR - 1))) * 16);
    b_off[i] = (uint32_t)(rb_ * g.ldb * EB) + b_kc[i];
  }
  const uint32_t a_pair = (uint32_t)uniform_i32(2 * RPC * g.lda * EB), b_pair = (uint32_t)uniform_i32(2 * RPC * g.ldb * EB);
  // DMA instruction i of operand A (isa) or B of stage st, into its ring's buffer. FULL: the stage
  // lies within K (stage offset in the scalar offset, no per-lane check); otherwise chunks past K
  // read zero.
  auto issue_one = [&](bool isa, int st, int i, bool FULL) __attribute__((always_inline)) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t kb = (uint32_t)st * BKB;
    const bool tail = !FULL && kb + BKB > KB;
    lds_ptr_t d = (lds_ptr_t)(isa ? sA(st % NSA) + (wave * A_CH + i) * 1024 : sB(st % NSB) + (wave * B_CH + i) * 1024);
    const uint32_t rs = (uint32_t)(i >> 1) * (isa ? a_pair : b_pair);
    const uint32_t vo = isa ? a_off[i & 1] : b_off[i & 1];
    if (FULL) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isa ? ra : rb, d, 16, vo, kb + rs, 0, 0);
    } else {
      uint32_t off = vo + rs + kb;
      if (tail && kb + (isa ? a_kc[i & 1] : b_kc[i & 1]) >= KB) off = 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isa ? ra : rb, d, 16, off, 0, 0, 0);
    }
#endif
  };

  acc_t acc[TT][TT];
#pragma unroll
  for (int i = 0; i < TT; ++i)
#pragma unroll
    for (int j = 0; j < TT; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[i][j][v] = 0;

  // Fragment reads: lane (fr, kq) reads chunk (4 kk + kq) of row fr of each 16-row tile, found at
  // slot chunk ^ swz(fr) (tile rows start at multiples of 16, so swz depends on fr only).
  const int fr = lane & 15, kq = lane >> 4;
  const int swz = (fr >> 1) & (CPR - 1);
  const int a_row = (wm * 128 + fr) * BKB, b_row = (wn * 128 + fr) * BKB;
  i32x4_t fa[2][TT], fb[2][TT];

  const int nst = (int)((KB + BKB - 1) / BKB);
  const int nsteps = nst * KST;
  // DMA order: the prologue issues A0 B0 A1 B1 .. (A up to NSA - 1, B up to NSB - 1); then, after
  // the readiness barrier of stage u + 1, B(u + NSB) and A(u + NSA), in that order. Stage u is
  // complete once only DMAs issued after both of its halves are outstanding: for u >= 1 that is
  // A(u + 1) when A runs a stage further ahead than B (issued right after B(u)); for u = 0 the
  // rest of the prologue.
  auto stage_ready = [&](int u, bool STEADY) __attribute__((always_inline)) {
    int ahead;
    if (u == 0)
      ahead = (nst > 1 ? A_CH + B_CH : 0) + (NSA > 2 && nst > 2 ? A_CH : 0);
    else
      ahead = (NSA > NSB && (STEADY || u + 1 < nst)) ? A_CH : 0;
    if (ahead >= 3 * A_CH)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(3 * A_CH));
    else if (ahead == 2 * A_CH)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(2 * A_CH));
    else if (ahead == A_CH)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(A_CH));
    else
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
  };

  for (int st = 0; st < NSA; ++st) {
    if (st < nst) {
#pragma unroll
      for (int q = 0; q < A_CH; ++q) issue_one(true, st, q, false);
    }
    if (st < NSB && st < nst) {
#pragma unroll
      for (int q = 0; q < B_CH; ++q) issue_one(false, st, q, false);
    }
  }
  stage_ready(0, false);
  {
    const int sl = (kq ^ swz) * 16;
#pragma unroll
    for (int i = 0; i < TT; ++i) fa[0][i] = *(const i32x4_t*)(sA(0) + a_row + sl + i * 16 * BKB);
#pragma unroll
    for (int j = 0; j < TT; ++j) fb[0][j] = *(const i32x4_t*)(sB(0) + b_row + sl + j * 16 * BKB);
  }

  // k-step t (fragments in parity P): its 64 MFMAs in 16 groups of four, each group preceded by
  // one fragment read of step t + 1 and, while refilling, one DMA instruction (B's first: it runs
  // one stage ahead, A NSA - 1). Crossing into a new stage, the step first passes that stage's
  // readiness barrier, which also frees the buffers of the stage just read, so their refills are
  // issued during the step. STEADY: every stage touched is full and both refills exist.
  auto step = [&](int t, int P, bool STEADY) __attribute__((always_inline)) {
    const int s = t / KST, kk = t - s * KST;
    const bool cross = kk + 1 == KST;  // the next k-step is in the next stage
    const bool next = !cross || STEADY || t + 1 < nsteps;
    const bool dma_b = cross && next && (STEADY || s + NSB < nst);
    const bool dma_a = cross && next && (STEADY || s + NSA < nst);
    if (cross && next) stage_ready(s + 1, STEADY);
    const int u = cross ? s + 1 : s, nkk = cross ? 0 : kk + 1;
    const int sl = ((4 * nkk + kq) ^ swz) * 16;
    const uint8_t* a_s = sA(u % NSA) + a_row + sl;
    const uint8_t* b_s = sB(u % NSB) + b_row + sl;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
      if (next) {
        if (q < TT)
          fb[P ^ 1][q] = *(const i32x4_t*)(b_s + q * 16 * BKB);
        else
          fa[P ^ 1][q - TT] = *(const i32x4_t*)(a_s + (q - TT) * 16 * BKB);
      }
      if (q < B_CH) {
        if (dma_b) issue_one(false, s + NSB, q, STEADY);
      } else {
        if (dma_a) issue_one(true, s + NSA, q - B_CH, STEADY);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = q >> 1, j = 4 * (q & 1) + e;
        MM::mma(acc[i][j], fb[P][j], fa[P][i]);
      }
    }
  };
  // Steady k-steps: the refills they issue are of full stages before the last (s + NSA <= nst - 2).
  int t = 0;
  const int steady_end = (nst - NSA - 1) * KST;
  for (; t + 1 < steady_end; t += 2) {
    step(t, 0, true);
    step(t + 1, 1, true);
  }
  for (; t + 1 < nsteps; t += 2) {
    step(t, 0, false);
    step(t + 1, 1, false);
  }
  if (t < nsteps) step(t, 0, false);
  // the last MFMAs' results before any read of the accumulators (their latency is not modelled)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  // Epilogue: lane holds row fr of MFMA tile (i, j), columns 16 j + 4 kq + 0..3. Tiles are taken in
  // pairs (j, j + 1), each accumulator read once. 16-bit outputs of a wave tile inside C are
  // regrouped between lanes kq and kq ^ 1 (v_permlane16_swap): an even kq stores columns
  // 16 j + 4 kq + 0..7, an odd kq columns 16 (j + 1) + 4 (kq - 1) + 0..7, one 16-byte store each.
  const int64_t cb = g.c_batch * batch;
  out_t* C = (out_t*)g.c;
  constexpr int OB = (int)sizeof(out_t);
  const int64_t wr0 = m0 + wm * 128, wc0 = n0 + wn * 128;
  const bool inside = wr0 + 128 <= g.M && wc0 + 128 <= g.N && g.ldc_n == 1 && g.ldc_m % 8 == 0 && cb % 8 == 0 &&
                      ((uintptr_t)g.c % 16) == 0 && (OUT != 4 || ((uintptr_t)g.scale % 16) == 0);
  const bool wide = OB == 2 && inside && (OUT != 4 || !g.acc_out);
  const bool odd = kq & 1;
  static_for<0, TT * TT / 2>([&](auto P) {
    constexpr int i = decltype(P)::value / (TT / 2), j = 2 * (decltype(P)::value % (TT / 2));
    const int64_t row = wr0 + 16 * i + fr;
    {
      // one tile pair at a time: the scheduler would otherwise hoist every accumulator read
      __builtin_amdgcn_sched_barrier(0);
      acc_t t2[2] = {acc[i][j], acc[i][j + 1]};
      if (wide) {
        uint32_t w[2][2];
#pragma unroll
        for (int d = 0; d < 2; ++d) {
          float sc[4] = {0.f, 0.f, 0.f, 0.f};
          if constexpr (OUT == 4) {
            const f32x4_t s4 = *(const f32x4_t*)(g.scale + wc0 + 16 * (j + d) + 4 * kq);
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[e] = s4[e];
          }
          if constexpr (OUT == 0 || OUT == 4) {
            w[d][0] = cvt_pair16<OUT>(t2[d], 0, sc[0], sc[1]);
            w[d][1] = cvt_pair16<OUT>(t2[d], 2, sc[2], sc[3]);
          } else {
            uint16_t o4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) o4[e] = (uint16_t)cvt4<OUT>(t2[d], e, sc[e]);
            const i32x2_t v2 = __builtin_bit_cast(i32x2_t, o4);
            w[d][0] = (uint32_t)v2[0];
            w[d][1] = (uint32_t)v2[1];
          }
        }
        // even lanes send tile j + 1, odd lanes tile j; each receives its partner's
        const uint32_t keep0 = odd ? w[1][0] : w[0][0], keep1 = odd ? w[1][1] : w[0][1];
        const uint32_t send0 = odd ? w[0][0] : w[1][0], send1 = odd ? w[0][1] : w[1][1];
        const auto r0 = __builtin_amdgcn_permlane16_swap(send0, send0, false, false);
        const auto r1 = __builtin_amdgcn_permlane16_swap(send1, send1, false, false);
        const uint32_t got0 = odd ? (uint32_t)r0[0] : (uint32_t)r0[1];
        const uint32_t got1 = odd ? (uint32_t)r1[0] : (uint32_t)r1[1];
        const i32x4_t q4 = odd ? i32x4_t{(int)got0, (int)got1, (int)keep0, (int)keep1}
                               : i32x4_t{(int)keep0, (int)keep1, (int)got0, (int)got1};
        const int64_t col = wc0 + 16 * j + (odd ? 16 + 4 * (kq - 1) : 4 * kq);
        *(i32x4_t*)((uint16_t*)C + cb + row * g.ldc_m + col) = q4;
        return;
      }
      if (row >= g.M) return;
#pragma unroll
      for (int d = 0; d < 2; ++d) {
        const int64_t col = wc0 + 16 * (j + d) + 4 * kq;
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        const bool vec4 = g.ldc_n == 1 && col + 3 < g.N && ((cb + row * g.ldc_m + col) * OB) % (4 * OB) == 0 &&
                          ((uintptr_t)g.c % (4 * OB)) == 0;
        if (vec4) {
          if constexpr (OUT == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[e] = g.scale[col + e];
          }
          out_t o4[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o4[e] = cvt4<OUT>(t2[d], e, sc[e]);
          const int64_t off = cb + row * g.ldc_m + col;
          if constexpr (OB == 1) {
            *(uint32_t*)(C + off) = __builtin_bit_cast(uint32_t, o4);
          } else if constexpr (OB == 2) {
            *(i32x2_t*)(C + off) = __builtin_bit_cast(i32x2_t, o4);
          } else {
            *(i32x4_t*)(C + off) = __builtin_bit_cast(i32x4_t, o4);
          }
          if constexpr (OUT == 4) {
            if (g.acc_out) *(i32x4_t*)(g.acc_out + off) = __builtin_bit_cast(i32x4_t, t2[d]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (col + e >= g.N) continue;
            if constexpr (OUT == 4) sc[e] = g.scale[col + e];
            const int64_t off = cb + row * g.ldc_m + (col + e) * g.ldc_n;
            C[off] = cvt4<OUT>(t2[d], e, sc[e]);
            if constexpr (OUT == 4) {
              if (g.acc_out) g.acc_out[off] = (int32_t)t2[d][e];
            }
          }
        }
      }
    }
  });
}

template <int KIND, int OUT, int NSA>
void gemm4_launch_cfg(hipStream_t s, const GemmDesc& d, void* c, const void* a, const void* b, const float* scale,
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
  g.tiles_m = (int)((d.M + 255) / 256);
  g.tiles_n = (int)((d.N + 255) / 256);
  const size_t lds = (size_t)(NSA + 2) * 256 * 128;
  static bool attr_set = false;
  if (!attr_set) {
    FO_HIP(hipFuncSetAttribute((const void*)k_gemm4<KIND, OUT, NSA>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)lds));
    attr_set = true;
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)d.batch);
  hipLaunchKernelGGL((k_gemm4<KIND, OUT, NSA>), grid, dim3(256), lds, s, g);
  FO_HIP(hipGetLastError());
}

template <int KIND, int OUT, int BM, int BN, int WM, int WN>
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
  size_t lds = (size_t)kNS * (BM + BN) * kRB;
  static bool attr_set = false;  // gfx950 LDS is 160 KiB; dynamic LDS above 64 KiB must be opted into
  if (!attr_set) {
    FO_HIP(hipFuncSetAttribute((const void*)k_gemm<KIND, OUT, BM, BN, WM, WN>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_set = true;
  }
  dim3 grid((unsigned)(g.tiles_m * g.tiles_n), (unsigned)d.batch);
  hipLaunchKernelGGL((k_gemm<KIND, OUT, BM, BN, WM, WN>), grid, dim3(64 * WM * WN), lds, s, g);
  FO_HIP(hipGetLastError());
}

// Tile choice: 256x256 when the problem is large -- four waves of 128x128 in 16x16 MFMA tiles
// (k_gemm4) for bf16 and i8 (plain outputs and the W8A8 dequant), eight waves of 128x64 in 32x32
// tiles (k_gemm) for the 8-bit floats -- and 128x128 otherwise. FO_GEMM_TILE overrides it for
// measurement: 128, 256 (k_gemm, 4 waves of 128x128), 2568 (8 waves of 128x64), 25616 (16 waves)
// or 4128 (k_gemm4).
template <int KIND, int OUT>
void gemm_launch(hipStream_t s, const GemmDesc& d, void* c, const void* a, const void* b,
                 const float* scale = nullptr, int32_t* acc_out = nullptr) {
  static int forced = [] {
    const char* e = getenv("FO_GEMM_TILE");
    return e ? atoi(e) : 0;
  }();
  int64_t tiles256 = ((d.M + 255) / 256) * ((d.N + 255) / 256) * d.batch;
  // Large problems: 8 waves of 128x64 for every kind: bf16 1-1.5% above 16 waves of 64x64 at
  // 4096^3 (same boxes, 200-launch runs); the 8-bit floats' 32-byte fragments make 16 waves of
  // 64x64 exceed 128 VGPRs and spill (1850 TFLOP/s against 367); i8 (the W8A8 config) 2175-2186
  // against 2135-2142 TOP/s with the refill split in parts.
  constexpr bool k16 = (KIND == kBf16 || KIND == kI8) && OUT <= 4;  // kinds with a 16x16 MFMA form here
  // Four waves of 128x128 for every kind with a 16x16 form: bf16 1258-1273 (eight-wave) against 1319
  // TFLOP/s, i8 -> i32 1660 against 1930 TOP/s, the W8A8 dequant 2432-2442 against 2490 TOP/s (same
  // boxes; before the four-wave kernel's refill interleave the W8A8 measured the other way round).
  constexpr bool k16_default = k16;
  int choice = forced ? forced : (tiles256 >= 128 ? (k16_default ? 4128 : 2568) : 128);
  if constexpr (k16) {
    // four waves of 128x128 (16x16 MFMA tiles), 128-byte stages, A and B double-buffered. (A
    // triple-buffered, running a stage further ahead than B in the 32 KiB of LDS left over, measured
    // 1030-1034 against 1300-1307 TFLOP/s on one box: correct, and slower.)
    if (choice == 4128) return gemm4_launch_cfg<KIND, OUT, 2>(s, d, c, a, b, scale, acc_out);
  }
  if (choice == 2568) return gemm_launch_cfg<KIND, OUT, 256, 256, 2, 4>(s, d, c, a, b, scale, acc_out);
  if (choice == 25616) return gemm_launch_cfg<KIND, OUT, 256, 256, 4, 4>(s, d, c, a, b, scale, acc_out);
  if (choice == 256) return gemm_launch_cfg<KIND, OUT, 256, 256, 2, 2>(s, d, c, a, b, scale, acc_out);
  return gemm_launch_cfg<KIND, OUT, 128, 128, 2, 2>(s, d, c, a, b, scale, acc_out);
}

}  // namespace

bool gemm_aligned(const void* a, const void* b, fo_dtype in_t, const GemmDesc& d) {
  int64_t eb = dtype_bytes(in_t);
  return ((uintptr_t)a % 16) == 0 && ((uintptr_t)b % 16) == 0 && (d.lda * eb) % 16 == 0 && (d.ldb * eb) % 16 == 0 &&
         (d.K * eb) % 16 == 0 && (d.a_batch * eb) % 16 == 0 && (d.b_batch * eb) % 16 == 0 && d.M < (1ll << 31) &&
         d.N < (1ll << 31) && d.batch < 65536;
}

bool gemm_supported(fo_dtype in_t, fo_dtype out_t) {
  return (in_t == FO_BF16 && (out_t == FO_BF16 || out_t == FO_F32)) ||
         (in_t == FO_I8 && (out_t == FO_I8 || out_t == FO_I32)) ||
         ((in_t == FO_F8E4M3 || in_t == FO_F8E5M2) && (out_t == in_t || out_t == FO_F32));
}

void launch_gemm(hipStream_t s, void* c, const void* a, const void* b, fo_dtype in_t, fo_dtype out_t,
                 const GemmDesc& d) {
  // 16-byte fragment loads need 16-byte aligned rows.
  require(gemm_aligned(a, b, in_t, d), "gemm: operands not 16-byte aligned or shape too large");
  if (in_t == FO_BF16 && out_t == FO_BF16) return gemm_launch<kBf16, 0>(s, d, c, a, b);
  if (in_t == FO_BF16 && out_t == FO_F32) return gemm_launch<kBf16, 1>(s, d, c, a, b);
  if (in_t == FO_I8 && out_t == FO_I8) return gemm_launch<kI8, 2>(s, d, c, a, b);
  if (in_t == FO_I8 && out_t == FO_I32) return gemm_launch<kI8, 3>(s, d, c, a, b);
  if (in_t == FO_F8E4M3 && out_t == FO_F8E4M3) return gemm_launch<kF8E4M3, 5>(s, d, c, a, b);
  if (in_t == FO_F8E4M3 && out_t == FO_F32) return gemm_launch<kF8E4M3, 1>(s, d, c, a, b);
  if (in_t == FO_F8E5M2 && out_t == FO_F8E5M2) return gemm_launch<kF8E5M2, 6>(s, d, c, a, b);
  if (in_t == FO_F8E5M2 && out_t == FO_F32) return gemm_launch<kF8E5M2, 1>(s, d, c, a, b);
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
  gemm_launch<kI8, 4>(s, d, out, a, w, scale, acc_out);
}

}  // namespace fo
