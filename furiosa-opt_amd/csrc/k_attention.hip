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
// MFMA layout. Each wave owns 32 queries. S^T = K Q^T is computed with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS, B = Q fragments held in registers for the whole kernel), so the
// accumulator gives every lane one query (lane % 32) and 16 keys per 32-key tile. Those registers
// are exactly the B operand of O^T = V^T P^T once the MFMA's k slots are bound to the keys the
// lane already holds (k order inside one MFMA is free as long as A and B agree): no shuffle of P
// through LDS. V is stored transposed in LDS with the keys of each 16-key group permuted so that
// every A fragment of the PV product is one 16-byte read.
//
// Pipeline. K and V tiles are double-buffered in LDS: the global loads for block j+1 are issued
// into registers before block j's MFMAs and written to the other LDS buffer after them, so one
// barrier per 64-key block suffices. Blocks entirely below the diagonal skip the mask; the O
// rescale is skipped when no query's running max moved.
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

constexpr int kBM = 128;  // queries per workgroup (4 waves x 32)
constexpr int kBN = 64;   // keys per block
constexpr float kEps = 6.25e-8f;  // attention.rs:13
constexpr float kL2E = 1.4426950408889634f;

__device__ __forceinline__ f32x16_t mma(const i32x4_t& a, const i32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
                                                 0, 0);
}

// Two f32 -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

template <int D>
struct AttnCfg {
  static constexpr int KROW = D * 2 + 16;    // bytes per K row in LDS (padded)
  static constexpr int VROW = kBN * 2 + 16;  // bytes per V^T row (one d) in LDS (padded)
  static constexpr int KBYTES = kBN * KROW;
  static constexpr int STAGE = KBYTES + D * VROW;
  static constexpr int LDS = 2 * STAGE;
  static constexpr int CH = D / 8;                        // 16-byte chunks per row
  static constexpr int KL = kBN * CH / 256;               // K chunks per thread
  static constexpr int VG = kBN / 4 * CH;                 // (4-key group, chunk) pairs per block
  static constexpr int VL = (VG + 255) / 256;             // such pairs per thread
  static constexpr int KS = D / 16;                       // k-steps of the QK^T contraction
  static constexpr int DT = D / 32;                       // 32-row d tiles of O^T
};

// Position of key `kk` (within a block) in a V^T row: inside each 16-key group, key 8h + 4g + i
// sits at 8g + 4h + i, so lane group g's two 4-key runs of a PV fragment are adjacent.
__device__ __forceinline__ int vt_pos(int kk) { return (kk & ~15) + ((kk & 4) << 1) + ((kk & 8) >> 1) + (kk & 3); }

template <int D, bool MASK>
__device__ __forceinline__ void attn_block(const uint8_t* __restrict__ sK, const uint8_t* __restrict__ sVt,
                                           const i32x4_t (&qf)[AttnCfg<D>::KS], f32x16_t (&o)[AttnCfg<D>::DT],
                                           float& m_run, float& l_part, int kv0, int myq, int seq, int causal,
                                           float inv_sd, int g, int col) {
  using C = AttnCfg<D>;
  f32x16_t s[2];
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
  // Logits: scale, round to bf16 (the reference's qk_scaled narrow), mask, block max.
  float bmax = -INFINITY;
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      uint32_t w = pack_bf16(s[kt][r] * inv_sd, s[kt][r + 1] * inv_sd);
      float x0 = __builtin_bit_cast(float, w << 16), x1 = __builtin_bit_cast(float, w & 0xffff0000u);
      if (MASK) {
        int key = kv0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        x0 = (key >= seq || (causal && key > myq)) ? -INFINITY : x0;
        x1 = (key + 1 >= seq || (causal && key + 1 > myq)) ? -INFINITY : x1;
      }
      s[kt][r] = x0;
      s[kt][r + 1] = x1;
      bmax = fmaxf(bmax, fmaxf(x0, x1));
    }
  bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
  const float m_new = fmaxf(m_run, bmax);
  const float ms = (m_new == -INFINITY) ? 0.f : m_new * kL2E;  // all-masked so far: keep p = 0, no NaN
  const float alpha = __builtin_amdgcn_exp2f(__builtin_fmaf(m_run, kL2E, -ms));
  m_run = m_new;
  // p = exp(x - m) as f32 for the sum, bf16 pairs for the PV operand. Chunk c = (kt = c/2,
  // h = c%2) holds s[kt][8h .. 8h+7].
  float psum = 0.f;
  i32x4_t pf[4];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][8 * h + 2 * e], kL2E, -ms));
        float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][8 * h + 2 * e + 1], kL2E, -ms));
        psum += p0 + p1;
        pf[kt * 2 + h][e] = (int)pack_bf16(p0, p1);
      }
  l_part = l_part * alpha + psum;
  if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {  // wave-uniform: some query's max moved
#pragma unroll
    for (int t = 0; t < C::DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
  }
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

template <int D>
__global__ void __launch_bounds__(256, 2) k_attn_fwd(uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
                                                     const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                     int32_t heads_total, int32_t seq, int32_t nqb, float inv_sd,
                                                     int32_t causal) {
  using C = AttnCfg<D>;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int bid = blockIdx.x;
  const int qb = nqb - 1 - bid / heads_total;  // heaviest (latest) query blocks first
  const int64_t head = bid % heads_total;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 5, col = lane & 31;
  const int q0 = qb * kBM;
  const int q0w = q0 + wave * 32;
  const int myq = q0w + col;

  const uint16_t* Qh = q + head * (int64_t)seq * D;
  const uint16_t* Kh = k + head * (int64_t)seq * D;
  const uint16_t* Vh = v + head * (int64_t)seq * D;

  // Q fragments (B operand of S^T): lane holds query myq, d in [16*ks + 8*g, +8).
  i32x4_t qf[C::KS];
#pragma unroll
  for (int ks = 0; ks < C::KS; ++ks) {
    if (myq < seq)
      qf[ks] = *(const i32x4_t*)(Qh + (int64_t)myq * D + ks * 16 + g * 8);
    else
      qf[ks] = i32x4_t{0, 0, 0, 0};
  }

  // Tile loaders. K: chunk c -> row c / CH, 16-byte column c % CH. V: pair p -> 4-key group
  // p % 16, column p / 16 (consecutive lanes take consecutive key groups, which keeps the
  // transposed 8-byte LDS writes of one instruction on distinct banks).
  i32x4_t kreg[C::KL];
  i32x4_t vreg[C::VL][4];
  auto load = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < C::KL; ++i) {
      int c = tid + i * 256, r = c / C::CH, cc = c % C::CH;
      kreg[i] = (kv0 + r < seq) ? *(const i32x4_t*)(Kh + (int64_t)(kv0 + r) * D + cc * 8) : i32x4_t{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < C::VL; ++i) {
      int p = tid + i * 256;
      if (C::VG % 256 != 0 && p >= C::VG) break;
      int kg = p % (kBN / 4), cc = p / (kBN / 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        int key = kv0 + kg * 4 + j;
        vreg[i][j] = (key < seq) ? *(const i32x4_t*)(Vh + (int64_t)key * D + cc * 8) : i32x4_t{0, 0, 0, 0};
      }
    }
  };
  auto store = [&](int buf) {
    uint8_t* sK = lds + buf * C::STAGE;
    uint8_t* sVt = sK + C::KBYTES;
#pragma unroll
    for (int i = 0; i < C::KL; ++i) {
      int c = tid + i * 256, r = c / C::CH, cc = c % C::CH;
      *(i32x4_t*)(sK + r * C::KROW + cc * 16) = kreg[i];
    }
#pragma unroll
    for (int i = 0; i < C::VL; ++i) {
      int p = tid + i * 256;
      if (C::VG % 256 != 0 && p >= C::VG) break;
      int kg = p % (kBN / 4), cc = p / (kBN / 4);
      int pos = vt_pos(kg * 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // d = cc*8 + e: keys 4kg .. 4kg+3 of that column, as two packed pairs.
        uint32_t a0 = (uint32_t)vreg[i][0][e >> 1], a1 = (uint32_t)vreg[i][1][e >> 1];
        uint32_t a2 = (uint32_t)vreg[i][2][e >> 1], a3 = (uint32_t)vreg[i][3][e >> 1];
        uint32_t w0, w1;
        if (e & 1) {
          w0 = (a0 >> 16) | (a1 & 0xffff0000u);
          w1 = (a2 >> 16) | (a3 & 0xffff0000u);
        } else {
          w0 = (a0 & 0xffffu) | (a1 << 16);
          w1 = (a2 & 0xffffu) | (a3 << 16);
        }
        *(i32x2_t*)(sVt + (cc * 8 + e) * C::VROW + pos * 2) = i32x2_t{(int)w0, (int)w1};
      }
    }
  };

  f32x16_t o[C::DT];
#pragma unroll
  for (int t = 0; t < C::DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;

  const int kv_end = causal ? min(seq, q0 + kBM) : seq;
  const int nblk = (kv_end + kBN - 1) / kBN;
  load(0);
  store(0);
  __syncthreads();
  for (int j = 0; j < nblk; ++j) {
    const int kv0 = j * kBN;
    const bool more = j + 1 < nblk;
    if (more) load(kv0 + kBN);
    const uint8_t* sK = lds + (j & 1) * C::STAGE;
    const uint8_t* sVt = sK + C::KBYTES;
    if (!(causal && kv0 > q0w + 31)) {  // wave-uniform: some of this wave's queries see these keys
      const bool need_mask = (causal && kv0 + kBN - 1 > q0w) || kv0 + kBN > seq;
      if (need_mask)
        attn_block<D, true>(sK, sVt, qf, o, m_run, l_part, kv0, myq, seq, causal, inv_sd, g, col);
      else
        attn_block<D, false>(sK, sVt, qf, o, m_run, l_part, kv0, myq, seq, causal, inv_sd, g, col);
    }
    if (more) store((j + 1) & 1);
    __syncthreads();
  }

  // out[myq][d] = bf16( bf16(o) / (l + EPS) ); lane holds d = 32t + 8*(r/4) + 4g + r%4.
  const float l_run = l_part + __shfl_xor(l_part, 32, 64);
  if (myq < seq) {
    const float denom = l_run + kEps;
    uint16_t* orow = out + head * (int64_t)seq * D + (int64_t)myq * D;
#pragma unroll
    for (int t = 0; t < C::DT; ++t)
#pragma unroll
      for (int blk = 0; blk < 4; ++blk) {
        i32x2_t w;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float a = bf16_to_f32(f32_to_bf16(o[t][blk * 4 + 2 * e]));
          float b = bf16_to_f32(f32_to_bf16(o[t][blk * 4 + 2 * e + 1]));
          uint32_t lo = f32_to_bf16(__fdiv_rn(a, denom)), hi = f32_to_bf16(__fdiv_rn(b, denom));
          w[e] = (int)(lo | (hi << 16));
        }
        *(i32x2_t*)(orow + t * 32 + 8 * blk + 4 * g) = w;
      }
  }
}

template <int D>
void launch_d(hipStream_t s, dim3 grid, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
              int64_t ht, int64_t seq, int64_t nqb, float inv_sd, int causal) {
  constexpr int lds = AttnCfg<D>::LDS;
  static bool attr_set = false;  // dynamic LDS above 64 KiB must be opted into
  if (!attr_set) {
    FO_HIP(hipFuncSetAttribute((const void*)k_attn_fwd<D>, hipFuncAttributeMaxDynamicSharedMemorySize, lds));
    attr_set = true;
  }
  hipLaunchKernelGGL(k_attn_fwd<D>, grid, dim3(256), lds, s, out, q, k, v, (int32_t)ht, (int32_t)seq, (int32_t)nqb,
                     inv_sd, causal);
}

}  // namespace

void launch_attention_prefill(hipStream_t s, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              int64_t batch, int64_t heads, int64_t seq, int64_t head_dim, float sqrt_d, int causal) {
  require(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0, "attention: buffers not aligned");
  int64_t ht = batch * heads;
  int64_t nqb = (seq + kBM - 1) / kBM;
  require(ht * nqb < (1ll << 31) && seq < (1ll << 30), "attention: shape too large");
  dim3 grid((unsigned)(ht * nqb));
  const float inv_sd = 1.0f / sqrt_d;
  if (head_dim == 128)
    launch_d<128>(s, grid, out, q, k, v, ht, seq, nqb, inv_sd, causal);
  else
    launch_d<64>(s, grid, out, q, k, v, ht, seq, nqb, inv_sd, causal);
  FO_HIP(hipGetLastError());
}

}  // namespace fo
