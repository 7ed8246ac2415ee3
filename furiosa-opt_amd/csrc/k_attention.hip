// Causal attention prefill: the QK^T -> softmax -> PV chain of the reference attention kernel
// (furiosa-opt-examples/src/transformer/kernel/attention.rs:32-392) as one flash-style kernel.
// Reference rounding points kept: logits s = bf16(f32(q.k) / sqrt_d) (qk_scaled, :53-63);
// p = exp(s - max) in f32 (masked_exp, :98-134); the denominator sums the f32 p plus EPS
// (row_sum, :137-156); PV multiplies bf16(p) (weighted_sum's cast, :167-176) with f32
// accumulation and narrows to bf16; the final division by the sum is done on that bf16 value
// (norm, :370-392). The running max/sum/alpha rescale is the reference's chunked online softmax
// (forward, :252-365) applied per 64-key block instead of per 512-key chunk. The f32 q.k sums
// are MFMA-reassociated, so the kernel is held to a tolerance, not bit parity; within that it
// scales the logits by RN(1/sqrt_d) instead of dividing and evaluates exp as exp2 of a fused
// multiply-add, both within an f32 ulp of the reference's operation.
//
// Given row maxima (row_max, one f32 per query row): the reference subtracts one max per row, taken
// over every key before masking (attention.rs:77-95), and rounds bf16(p) at that scale. A running
// max rounds bf16(p) at another scale, and where a row's output is a near-cancelling average of
// thousands of values those roundings do not cancel. With row_max given, the reference max starts
// at the given value instead of -inf: for the reference's own max no block exceeds it, so no rescale
// happens and every p = exp(s - m) is the reference's, at most 1; p is then clipped at 1 as the
// reference's mask clip does, which changes only a NaN p (a NaN logit), into 1. The given value must
// be at least the max over the row's visible keys (the reference's max over every key is).
//
// Workgroups of kWaves = 8 waves (256 queries, two waves per SIMD) share each K/V tile: one load of
// it per 256 queries (measured 4% faster than two workgroups of four waves per CU).
//
// MFMA layout. Each wave owns 32 queries. S^T = K Q^T is computed with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS, B = Q fragments held in registers for the whole tile), so the
// accumulator gives every lane one query (lane % 32) and 16 keys per 32-key tile. Those registers
// are exactly the B operand of O^T = V^T P^T once the MFMA's k slots are bound to the keys the
// lane already holds (k order inside one MFMA is free as long as A and B agree): no shuffle of P
// through LDS. V is stored transposed in LDS with the keys of each 16-key group permuted so that
// every A fragment of the PV product is one 16-byte read.
//
// Pipeline. K and V tiles are double-buffered in LDS. A step computes S of its block, the
// softmax, then the PV product; the two waves that share a SIMD overlap one's MFMAs with the
// other's softmax. (Computing the next block's S during this block's softmax, in the same wave,
// measured 7% slower: the second S tile's 32 registers leave none for LDS reads in flight.)
// Global loads for the next block are issued into registers before a step and written to LDS
// after it, so one barrier per block suffices. Blocks below the last kBM / kBN are fully visible to
// every query of the workgroup and run without mask code; of the last ones, a wave runs the mask
// code only on a block that hides some key from one of its queries.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float f32x2_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2_t;

constexpr int kWaves = 8;          // waves per workgroup
constexpr int kNT = 64 * kWaves;    // threads per workgroup
constexpr int kBM = 32 * kWaves;    // queries per workgroup (32 per wave)
constexpr int kBN = 64;   // keys per block
constexpr float kEps = 6.25e-8f;  // attention.rs:13
constexpr float kL2E = 1.4426950408889634f;
constexpr float kTau = 5.545177444479562f;  // 8 ln 2: p = exp(s - m_run) <= 2^8 between rescales

__device__ __forceinline__ f32x16_t mma(const i32x4_t& a, const i32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
                                                 0, 0);
}

// The two values of lanes l and l ^ 32 (v_permlane32_swap: lanes below 32 get {own, l + 32},
// lanes from 32 get {l - 32, own}, so both halves see the pair in the same order).
struct LanePair {
  float lo, hi;
};
__device__ __forceinline__ LanePair half_pair(float v) {
  const uint32_t u = __builtin_bit_cast(uint32_t, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return {__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}

// Two 4-column bf16 groups of an MFMA output row (lanes l < 32 hold columns c + 0..3, lanes l + 32
// columns c + 4..7, for group a at c and group b at c + 8) regrouped across the wave halves: lane
// l < 32 gets columns c + 0..7 of its row, lane l + 32 columns c + 8..15, one 16-byte store each.
__device__ __forceinline__ i32x4_t regroup8(i32x2_t a, i32x2_t b) {
  const auto r0 = __builtin_amdgcn_permlane32_swap((uint32_t)a[0], (uint32_t)b[0], false, false);
  const auto r1 = __builtin_amdgcn_permlane32_swap((uint32_t)a[1], (uint32_t)b[1], false, false);
  return i32x4_t{(int)r0[0], (int)r1[0], (int)r0[1], (int)r1[1]};
}

// Two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// f32 -> bf16 (round to nearest even) -> f32 in one instruction: the bf16 lands in the high half of
// v_cvt_pk_bf16_f32's result above a zero low half, which read as f32 is the bf16 value itself
// (against a packed pair and two unpacking instructions for two values).
__device__ __forceinline__ float round_bf16(float x) { return __builtin_bit_cast(float, pack_bf16(0.f, x)); }

template <int D>
struct AttnCfg {
  static constexpr int KROW = D * 2 + 16;    // bytes per K row in LDS (padded)
  static constexpr int VROW = kBN * 2 + 16;  // bytes per V^T row (one d) in LDS (padded)
  static constexpr int KBYTES = kBN * KROW;
  static constexpr int STAGE = KBYTES + D * VROW;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int CH = D / 8;             // 16-byte chunks per row
  static constexpr int KL = kBN * CH / kNT;    // K chunks per thread
  static constexpr int VG = kBN / 4 * CH;      // (4-key group, chunk) pairs per block
  static constexpr int VL = (VG + kNT - 1) / kNT;  // such pairs per thread
  static constexpr int KS = D / 16;            // k-steps of the QK^T contraction
  static constexpr int DT = D / 32;            // 32-row d tiles of O^T
};

// Position of key `kk` (within a block) in a V^T row: inside each 16-key group, key 8h + 4g + i
// sits at 8g + 4h + i, so lane group g's two 4-key runs of a PV fragment are adjacent.
__device__ __forceinline__ int vt_pos(int kk) { return (kk & ~15) + ((kk & 4) << 1) + ((kk & 8) >> 1) + (kk & 3); }

// S^T tile pair for the 64 keys of one K buffer: keys kt*32 + 8*(r/4) + 4g + r%4 of s[kt][r].
template <int D>
__device__ __forceinline__ void qk(const uint8_t* __restrict__ sK, const i32x4_t (&qf)[AttnCfg<D>::KS],
                                   f32x16_t (&s)[2], int g, int col) {
  using C = AttnCfg<D>;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < C::KS; ++ks) {
      i32x4_t kf = *(const i32x4_t*)(sK + (kt * 32 + col) * C::KROW + ks * 32 + g * 16);
      s[kt] = mma(kf, qf[ks], s[kt]);
    }
  }
}

// One step: S of the block (K from sK), its softmax, then its PV product (V^T from sVt).
template <int D, bool MASK, bool GIVEN>
__device__ __forceinline__ void attn_step(const uint8_t* __restrict__ sK, const uint8_t* __restrict__ sVt,
                                          const i32x4_t (&qf)[AttnCfg<D>::KS], f32x16_t (&o)[AttnCfg<D>::DT],
                                          float& m_run, float& l_part,
                                          int kv0, int lim, float inv_sd, int g, int col) {
  using C = AttnCfg<D>;
  f32x16_t sc[2];
  qk<D>(sK, qf, sc, g, col);
  // Scaled sums first, then the block max over them (the max of products is the product of the
  // max, and bf16 rounding is monotonic, so the max commutes with both). Taking it on product
  // results also spares the quieting of each operand that a max of raw MFMA outputs needs.
  float bmax = -INFINITY, bmax2 = -INFINITY;
  float xs[2][16];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
    for (int r = 0; r < 16; ++r) xs[kt][r] = sc[kt][r] * inv_sd;
    if (MASK) {
      // key kv0 + kt*32 + 8(r/4) + 4g + r%4 is visible iff it is <= lim: one compare against a
      // per-lane threshold with the register's constant key offset.
      const int thr = lim - kv0 - kt * 32 - 4 * g;
#pragma unroll
      for (int r = 0; r < 16; ++r) xs[kt][r] = (8 * (r >> 2) + (r & 3) > thr) ? -INFINITY : xs[kt][r];
    }
#pragma unroll
    for (int r = 0; r < 16; r += 4) {  // two chains of three-way maxima
      bmax = __builtin_fmaxf(__builtin_fmaxf(bmax, xs[kt][r]), xs[kt][r + 1]);
      bmax2 = __builtin_fmaxf(__builtin_fmaxf(bmax2, xs[kt][r + 2]), xs[kt][r + 3]);
    }
  }
  bmax = __builtin_fmaxf(bmax, bmax2);
  {
    const LanePair b = half_pair(bmax);  // the query's other 32 keys live in lane ^ 32
    bmax = __builtin_fmaxf(b.lo, b.hi);
  }
  bmax = round_bf16(bmax);
  // Online softmax step with a lazy reference max: O and the sum are rescaled only when some
  // lane's block max exceeds its reference max by more than kTau, so p = exp(s - m_run) stays
  // <= e^kTau = 256 and most blocks skip the rescale of the 64 O registers. The ratio O / sum
  // does not depend on the reference (every p of a row shares it). Every query of a processed
  // block sees key 0 of the first block, so the first block always rescales (alpha = 0 there,
  // m_run = -inf) and m_run is finite from then on.
  if (bmax > m_run + kTau) {  // per lane: skipped as a whole when no lane of the wave needs it
    const float alpha = __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, kL2E, -bmax * kL2E));
    m_run = bmax;
    l_part *= alpha;
#pragma unroll
    for (int t = 0; t < C::DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
  }
  const float ms = m_run * kL2E;
  // p = exp(x - m) as f32 for the sum, bf16 pairs for the PV operand. Chunk c = (kt = c/2,
  // h = c%2) holds sc[kt][8h .. 8h+7].
  float psum = 0.f;
  i32x4_t pf[4];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 8 * h + 2 * e;
        const float x0 = round_bf16(xs[kt][r]), x1 = round_bf16(xs[kt][r + 1]);
        float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(x0, kL2E, -ms));
        float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(x1, kL2E, -ms));
        if (GIVEN) {
          // The reference's mask is vector_clip(Min, mask) on p (attention.rs:98-134): with the
          // reference's max every p <= 1 and min(p, 1) = p, while a NaN p (a NaN logit) becomes 1;
          // a masked key's p is min(p, 0) = 0 whatever p is (also where a row's max is -inf and
          // exp(-inf - m) is NaN).
          p0 = __builtin_fminf(p0, 1.0f);
          p1 = __builtin_fminf(p1, 1.0f);
          if (MASK) {
            const int thr = lim - kv0 - kt * 32 - 4 * g;
            p0 = (8 * (r >> 2) + (r & 3) > thr) ? 0.0f : p0;
            p1 = (8 * ((r + 1) >> 2) + ((r + 1) & 3) > thr) ? 0.0f : p1;
          }
        }
        psum += p0 + p1;
        pf[kt * 2 + h][e] = (int)pack_bf16(p0, p1);
      }
  l_part += psum;
  // O^T += V^T P^T. Chunk c covers keys base = 32*(c/2) + 16*(c%2); lane group g binds k slots to
  // keys {base + 4g + 0..3, base + 8 + 4g + 0..3}, stored adjacently at base + 8g.
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int base = 32 * (c >> 1) + 16 * (c & 1);
#pragma unroll
    for (int t = 0; t < C::DT; ++t) {
      i32x4_t vf = *(const i32x4_t*)(sVt + (t * 32 + col) * C::VROW + (base + 8 * g) * 2);
      o[t] = mma(vf, pf[c], o[t]);
    }
  }
}

template <int D, bool GIVEN>
__global__ void __launch_bounds__(kNT, 2 * 4 / kWaves) k_attn_fwd(uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
                                                     const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     const float* __restrict__ row_max, int32_t heads_total,
                                                     int32_t seq, int32_t nqb, float inv_sd, int32_t causal) {
  using C = AttnCfg<D>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int bid = blockIdx.x;
  // Heaviest (latest) query blocks first. Workgroups go to the XCDs round-robin, so a head whose
  // query blocks share bid % 8 keeps them on one XCD's L2: in groups of four query blocks, the
  // first 256 workgroups are blocks nqb - 1 .. nqb - 4 of half the heads, which start together and
  // read each K / V block within a short window (166.0 against 168.5 us, medians of five bench runs
  // each on one box, for blocks nqb - 1 and nqb - 2 of every head first).
  int qb = nqb - 1 - bid / heads_total;
  int64_t head = bid % heads_total;
  if (nqb % 4 == 0 && heads_total % 16 == 0) {
    const int H = heads_total, c = bid / (4 * H), r = bid % (4 * H), half = r / (2 * H), r2 = r % (2 * H);
    head = half * (H / 2) + r2 % (H / 2);
    qb = nqb - 1 - (4 * c + r2 / (H / 2));
  }
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform per wave: scalar branches
  const int g = lane >> 5, col = lane & 31;
  const int q0 = qb * kBM;
  const int q0w = q0 + wave * 32;
  const int myq = q0w + col;
  const int lim = causal ? min(myq, seq - 1) : seq - 1;  // last key this lane's query sees

  const uint16_t* Qh = q + head * (int64_t)seq * D;
  const uint16_t* Kh = k + head * (int64_t)seq * D;
  const uint16_t* Vh = v + head * (int64_t)seq * D;
  // Buffer loads bounded to the head's seq rows: rows past the end read as zero, so the tail
  // block and the queries past the end need no guards.
  const uint32_t head_bytes = (uint32_t)seq * D * 2;
  const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc((void*)Qh, (short)0, (int)head_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)Kh, (short)0, (int)head_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)Vh, (short)0, (int)head_bytes, 0x00020000);

  // Tile loaders. K: chunk c -> row c / CH, 16-byte column c % CH. V: pair p -> 4-key group
  // p % 16, column p / 16 (consecutive lanes take consecutive key groups, which keeps the
  // transposed 8-byte LDS writes of one instruction on distinct banks).
  const uint32_t koff = (uint32_t)(((tid / C::CH) * D + (tid % C::CH) * 8) * 2);
  const uint32_t voff = (uint32_t)((((tid % (kBN / 4)) * 4) * D + (tid / (kBN / 4)) * 8) * 2);
  i32x4_t kreg[C::KL];
  i32x4_t vreg[C::VL][4];
  auto load_k = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < C::KL; ++i)
      kreg[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff, kv0 * D * 2 + i * (kNT / C::CH) * D * 2, 0);
  };
  auto load_v = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < C::VL; ++i) {
      if (C::VG % kNT != 0 && tid + i * kNT >= C::VG) break;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        vreg[i][j] = __builtin_amdgcn_raw_buffer_load_b128(rv, voff + j * D * 2, kv0 * D * 2 + i * kNT / (kBN / 4) * 16, 0);
    }
  };
  auto store_k = [&](int buf) {
    uint8_t* sK = lds + buf * C::STAGE;
#pragma unroll
    for (int i = 0; i < C::KL; ++i) {
      int c = tid + i * kNT, r = c / C::CH, cc = c % C::CH;
      *(i32x4_t*)(sK + r * C::KROW + cc * 16) = kreg[i];
    }
  };
  auto store_v = [&](int buf) {
    uint8_t* sVt = lds + buf * C::STAGE + C::KBYTES;
#pragma unroll
    for (int i = 0; i < C::VL; ++i) {
      int p = tid + i * kNT;
      if (C::VG % kNT != 0 && p >= C::VG) break;
      int kg = p % (kBN / 4), cc = p / (kBN / 4);
      int pos = vt_pos(kg * 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // d = cc*8 + e: keys 4kg .. 4kg+3 of that column, as two packed pairs.
        uint32_t a0 = (uint32_t)vreg[i][0][e >> 1], a1 = (uint32_t)vreg[i][1][e >> 1];
        uint32_t a2 = (uint32_t)vreg[i][2][e >> 1], a3 = (uint32_t)vreg[i][3][e >> 1];
        // v_perm_b32 byte select over {hi = a1, lo = a0}: low halves 0x05040100, high 0x07060302.
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        uint32_t w0 = __builtin_amdgcn_perm(a1, a0, sel);
        uint32_t w1 = __builtin_amdgcn_perm(a3, a2, sel);
        *(i32x2_t*)(sVt + (cc * 8 + e) * C::VROW + pos * 2) = i32x2_t{(int)w0, (int)w1};
      }
    }
  };
  auto sK_of = [&](int buf) { return (const uint8_t*)(lds + buf * C::STAGE); };
  auto sVt_of = [&](int buf) { return (const uint8_t*)(lds + buf * C::STAGE + C::KBYTES); };

  // Prologue: Q fragments (B operand of S^T: lane holds query myq, d in [16*ks + 8*g, +8)), K(0)
  // and V(0) are requested together.
  i32x4_t qf[C::KS];
  const uint32_t qoff = (uint32_t)(myq * D + g * 8) * 2;
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) qf[ks] = __builtin_amdgcn_raw_buffer_load_b128(rq, qoff, ks * 32, 0);
  load_k(0);
  load_v(0);
  store_k(0);
  store_v(0);

  f32x16_t o[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;
  if (row_max && myq < seq) m_run = row_max[head * (int64_t)seq + myq];

  // Buffers: K(j) and V(j) live in buffer j % 2. Step j reads them, and after it writes K(j+1)
  // and V(j+1) (loaded during the step) into buffer (j+1) % 2, last read by step j-1 before the
  // previous barrier. Loads past the head's end read zeros, so every step loads and stores
  // unconditionally.
  const int kv_end = causal ? min(seq, q0 + kBM) : seq;
  const int nblk = (kv_end + kBN - 1) / kBN;
  const int nmain = nblk > kBM / kBN ? nblk - kBM / kBN : 0;
  __syncthreads();
  int j = 0;
  for (; j < nmain; ++j) {
    const int kv0 = j * kBN;
    load_k(kv0 + kBN);
    load_v(kv0 + kBN);
    __builtin_amdgcn_sched_barrier(0);
    attn_step<D, false, GIVEN>(sK_of(j & 1), sVt_of(j & 1), qf, o, m_run, l_part, kv0, lim, inv_sd, g, col);
    store_k((j + 1) & 1);
    store_v((j + 1) & 1);
    __syncthreads();
  }
  // In the last blocks a wave runs the mask code only where some key of the block is hidden from
  // one of its queries: blocks wholly visible to its first query (and inside the sequence) run
  // unmasked, blocks past its last query are skipped, so each wave masks one block of the diagonal
  // (and, without causality, the sequence's last) instead of every block up to it.
  const int vis = causal ? min(q0w, seq - 1) : seq - 1;  // last key every query of the wave sees
  for (; j < nblk; ++j) {
    const int kv0 = j * kBN;
    load_k(kv0 + kBN);
    load_v(kv0 + kBN);
    __builtin_amdgcn_sched_barrier(0);
    if (kv0 + kBN - 1 <= vis)  // wave-uniform
      attn_step<D, false, GIVEN>(sK_of(j & 1), sVt_of(j & 1), qf, o, m_run, l_part, kv0, lim, inv_sd, g, col);
    else if (!(causal && kv0 > q0w + 31))  // wave-uniform
      attn_step<D, true, GIVEN>(sK_of(j & 1), sVt_of(j & 1), qf, o, m_run, l_part, kv0, lim, inv_sd, g, col);
    store_k((j + 1) & 1);
    store_v((j + 1) & 1);
    __syncthreads();
  }

  // out[myq][d] = bf16( bf16(o) / (l + EPS) ); lane holds d = 32t + 8*(r/4) + 4g + r%4. The
  // quotient is correctly rounded (the divisor is normal: l >= 1 with the running max, l + EPS >=
  // EPS with a given one; |o| <= l max|v| keeps the quotient finite); both narrows are the
  // hardware's round-to-nearest-even (finite inputs give finite, normal-or-zero o).
  const LanePair lp = half_pair(l_part);
  const float l_run = lp.lo + lp.hi;
  // Every lane computes (a query past the end sees every key, so its l >= 1 too); lanes l and
  // l + 32 hold the same query row, so the regrouped 16-byte stores share one condition.
  const float denom = l_run + kEps;
  const float rinv = __fdiv_rn(1.0f, denom);
  uint16_t* orow = out + head * (int64_t)seq * D + (int64_t)myq * D;
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int bp = 0; bp < 4; bp += 2) {
      i32x2_t wv[2];
#pragma unroll
      for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int blk = bp + d;
          const uint32_t ob = pack_bf16(o[t][blk * 4 + 2 * e], o[t][blk * 4 + 2 * e + 1]);
          const float a = __builtin_bit_cast(float, ob << 16), b = __builtin_bit_cast(float, ob & 0xffff0000u);
          // An infinite o (an infinite value in V) divides to itself; div_cr's remainder would be NaN.
          const float qa = __builtin_isinf(a) ? a : div_cr(a, denom, rinv);
          const float qb = __builtin_isinf(b) ? b : div_cr(b, denom, rinv);
          wv[d][e] = (int)pack_bf16(qa, qb);
        }
      const i32x4_t q4 = regroup8(wv[0], wv[1]);
      if (myq < seq) *(i32x4_t*)(orow + t * 32 + 8 * bp + 8 * g) = q4;
    }
}

template <int D, bool GIVEN>
void launch_d(hipStream_t s, dim3 grid, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
              const float* row_max, int64_t ht, int64_t seq, int64_t nqb, float inv_sd, int causal) {
  constexpr int lds = AttnCfg<D>::LDS;
  static bool attr_set = false;  // dynamic LDS above 64 KiB must be opted into
  if (!attr_set) {
    FO_HIP(hipFuncSetAttribute((const void*)k_attn_fwd<D, GIVEN>, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    attr_set = true;
  }
  hipLaunchKernelGGL((k_attn_fwd<D, GIVEN>), grid, dim3(kNT), lds, s, out, q, k, v, row_max, (int32_t)ht, (int32_t)seq,
                     (int32_t)nqb, inv_sd, causal);
}

}  // namespace

void launch_attention_prefill(hipStream_t s, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const float* row_max, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                              float sqrt_d, int causal) {
  require(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0, "attention: buffers not aligned");
  int64_t ht = batch * heads;
  int64_t nqb = (seq + kBM - 1) / kBM;
  require(ht * nqb < (1ll << 31) && (seq + 2 * kBN) * head_dim * 2 < (1ll << 31), "attention: shape too large");
  dim3 grid((unsigned)(ht * nqb));
  const float inv_sd = 1.0f / sqrt_d;
  if (head_dim == 128)
    row_max ? launch_d<128, true>(s, grid, out, q, k, v, row_max, ht, seq, nqb, inv_sd, causal)
            : launch_d<128, false>(s, grid, out, q, k, v, row_max, ht, seq, nqb, inv_sd, causal);
  else
    row_max ? launch_d<64, true>(s, grid, out, q, k, v, row_max, ht, seq, nqb, inv_sd, causal)
            : launch_d<64, false>(s, grid, out, q, k, v, row_max, ht, seq, nqb, inv_sd, causal);
  FO_HIP(hipGetLastError());
}

}  // namespace fo
