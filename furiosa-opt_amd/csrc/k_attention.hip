// Causal attention prefill: the QK^T -> softmax -> PV chain of the reference attention kernel
// (furiosa-opt-examples/src/transformer/kernel/attention.rs:32-392) as one flash-style kernel.
// Reference rounding points kept: logits s = bf16(f32(q.k) / sqrt_d) (qk_scaled, :53-63);
// p = exp(s - max) in f32 (masked_exp, :98-134); the denominator sums the f32 p plus EPS
// (row_sum, :137-156); PV multiplies bf16(p) (weighted_sum's cast, :167-176) with f32
// accumulation and narrows to bf16; the final division by the sum is done on that bf16 value
// (norm, :370-392). The running max/sum/alpha rescale is the reference's chunked online softmax
// (forward, :252-365) applied per 64-key block instead of per 512-key chunk.
//
// MFMA layout. Each wave owns 32 queries. S^T = K Q^T is computed with v_mfma_f32_32x32x16_bf16
// (A = K rows from LDS, B = Q fragments held in registers for the whole kernel), so the
// accumulator gives every lane one query (lane % 32) and 16 keys per 32-key tile. Those registers
// are exactly the B operand of O^T = V^T P^T once the MFMA's k slots are bound to the keys the
// lane already holds (k order inside one MFMA is free as long as A and B agree): no shuffle of P
// through LDS. V is stored transposed in LDS so the A fragments are two 8-byte reads.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2_t;

constexpr int kBM = 128;  // queries per workgroup (4 waves x 32)
constexpr int kBN = 64;   // keys per block
constexpr float kEps = 6.25e-8f;  // attention.rs:13

__device__ __forceinline__ f32x16_t mma(const i32x4_t& a, const i32x4_t& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c, 0,
                                                 0, 0);
}

template <int D>
__global__ void __launch_bounds__(256) k_attn_fwd(uint16_t* __restrict__ out, const uint16_t* __restrict__ q,
                                                  const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                  int32_t heads_total, int32_t seq, int32_t nqb, float sqrt_d,
                                                  int32_t causal) {
  constexpr int KROW = D * 2 + 16;    // bytes per K row in LDS (padded)
  constexpr int VROW = kBN * 2 + 16;  // bytes per V^T row (one d) in LDS (padded)
  constexpr int KS = D / 16;          // k-steps of the QK^T contraction
  constexpr int DT = D / 32;          // 32-row d tiles of O^T
  __shared__ __attribute__((aligned(16))) uint8_t sK[kBN * KROW];
  __shared__ __attribute__((aligned(16))) uint8_t sVt[D * VROW];

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
  i32x4_t qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (myq < seq)
      qf[ks] = *(const i32x4_t*)(Qh + (int64_t)myq * D + ks * 16 + g * 8);
    else
      qf[ks] = i32x4_t{0, 0, 0, 0};
  }

  f32x16_t o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  int kv_end = causal ? min(seq, q0 + kBM) : seq;
  for (int kv0 = 0; kv0 < kv_end; kv0 += kBN) {
    __syncthreads();  // previous block's LDS reads are done
    // K tile: 64 keys x D, 16-byte chunks.
    constexpr int CH = D / 8;  // 16-byte chunks per row
    for (int c = tid; c < kBN * CH; c += 256) {
      int r = c / CH, cc = c % CH;
      i32x4_t val = i32x4_t{0, 0, 0, 0};
      if (kv0 + r < seq) val = *(const i32x4_t*)(Kh + (int64_t)(kv0 + r) * D + cc * 8);
      *(i32x4_t*)(sK + r * KROW + cc * 16) = val;
    }
    // V tile transposed: sVt[d][key].
    for (int c = tid; c < kBN * CH; c += 256) {
      int r = c / CH, cc = c % CH;
      i32x4_t val = i32x4_t{0, 0, 0, 0};
      if (kv0 + r < seq) val = *(const i32x4_t*)(Vh + (int64_t)(kv0 + r) * D + cc * 8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        uint32_t w = (uint32_t)val[e >> 1];
        uint16_t h = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
        *(uint16_t*)(sVt + (cc * 8 + e) * VROW + r * 2) = h;
      }
    }
    __syncthreads();
    if (causal && kv0 > q0w + 31) continue;  // this wave's queries see none of these keys

    // S^T tiles: keys kv0 + kt*32 + (8*(r/4) + 4*g + r%4), query myq.
    f32x16_t s[2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        i32x4_t kf = *(const i32x4_t*)(sK + (kt * 32 + col) * KROW + ks * 32 + g * 16);
        s[kt] = mma(kf, qf[ks], s[kt]);
      }
    }
    // Scale, round the logits to bf16, mask, block max.
    float bmax = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int key = kv0 + kt * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
        float x = bf16_to_f32(f32_to_bf16(__fdiv_rn(s[kt][r], sqrt_d)));
        bool dead = key >= seq || (causal && key > myq);
        x = dead ? -INFINITY : x;
        s[kt][r] = x;
        bmax = fmaxf(bmax, x);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    float m_new = fmaxf(m_run, bmax);
    float alpha = (m_run == -INFINITY) ? 0.f : __expf(m_run - m_new);
    float psum = 0.f;
    i32x4_t pf[4];  // bf16 P fragments: chunk c = (kt = c/2, half h = c%2) holds s[kt][8h .. 8h+7]
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float p0 = s[kt][8 * h + 2 * e] == -INFINITY ? 0.f : __expf(s[kt][8 * h + 2 * e] - m_new);
          float p1 = s[kt][8 * h + 2 * e + 1] == -INFINITY ? 0.f : __expf(s[kt][8 * h + 2 * e + 1] - m_new);
          psum += p0 + p1;
          uint32_t lo = f32_to_bf16(p0), hi = f32_to_bf16(p1);
          pf[kt * 2 + h][e] = (int)(lo | (hi << 16));
        }
      }
    psum += __shfl_xor(psum, 32, 64);
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
    // O^T += V^T P^T. Chunk c covers keys base = 32*(c/2) + 16*(c%2); lane group g supplies
    // k slots {base + 4g + 0..3, base + 8 + 4g + 0..3} -- the keys its P registers hold.
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int base = 32 * (c >> 1) + 16 * (c & 1);
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const uint8_t* row = sVt + (t * 32 + col) * VROW;
        i32x2_t lo = *(const i32x2_t*)(row + (base + 4 * g) * 2);
        i32x2_t hi = *(const i32x2_t*)(row + (base + 8 + 4 * g) * 2);
        i32x4_t vf = i32x4_t{lo[0], lo[1], hi[0], hi[1]};
        o[t] = mma(vf, pf[c], o[t]);
      }
    }
  }

  // out[myq][d] = bf16( bf16(o) / (l + EPS) ); lane holds d = 32t + 8*(r/4) + 4g + r%4.
  if (myq < seq) {
    float denom = l_run + kEps;
    uint16_t* orow = out + head * (int64_t)seq * D + (int64_t)myq * D;
#pragma unroll
    for (int t = 0; t < DT; ++t)
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

}  // namespace

void launch_attention_prefill(hipStream_t s, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              int64_t batch, int64_t heads, int64_t seq, int64_t head_dim, float sqrt_d, int causal) {
  require(((uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)out) % 16 == 0, "attention: buffers not aligned");
  int64_t ht = batch * heads;
  int64_t nqb = (seq + kBM - 1) / kBM;
  require(ht * nqb < (1ll << 31) && seq < (1ll << 30), "attention: shape too large");
  dim3 grid((unsigned)(ht * nqb));
  if (head_dim == 128)
    hipLaunchKernelGGL(k_attn_fwd<128>, grid, dim3(256), 0, s, out, q, k, v, (int32_t)ht, (int32_t)seq, (int32_t)nqb,
                       sqrt_d, causal);
  else
    hipLaunchKernelGGL(k_attn_fwd<64>, grid, dim3(256), 0, s, out, q, k, v, (int32_t)ht, (int32_t)seq, (int32_t)nqb,
                       sqrt_d, causal);
  FO_HIP(hipGetLastError());
}

}  // namespace fo
