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

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
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
    return f32_to_bf16(__fmul_rn(fixedpoint_to_float((int32_t)a[v], 31), sc));
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

// Tile choice: 256x256 with 8 waves of 128x64 (one tile per CU at 4096^2, two waves per SIMD)
// when the problem is large, 128x128 otherwise (measured best on MI355X among 128, 256 with 4, 8
// and 16 waves). FO_GEMM_TILE overrides it for measurement: 128, 256 (4 waves of 128x128),
// 2568 (8 waves of 128x64) or 25616 (16 waves).
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
  int choice = forced ? forced : (tiles256 >= 128 ? 2568 : 128);
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
