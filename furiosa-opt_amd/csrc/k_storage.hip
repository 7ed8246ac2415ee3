// gfx950 kernels for the mapping-driven storage ops of the Backend seam:
//   relayout   BufStorage::transpose      (storage/buf.rs:257-313)
//   transmute  BufStorage::transmute      (storage/buf.rs:592-601)
//   map/zip    BufStorage::map/zip_with/zip3_with (storage/buf.rs:203-250) with the VE op set
//              (engine/vector/op/semantics.rs) and apply_slots (vector_tensor.rs:892-938)
//   reduce     BufStorage::reduce         (storage/buf.rs:331-376)
//   contraction_in generic fold           (storage/buf.rs:401-447)
// Every odometer is walked with 32-bit magic-number division; memory offsets are 64-bit.
#include <hip/hip_runtime.h>

#include "runtime.hpp"

namespace fo {
namespace {

constexpr int kBlock = 256;

inline int grid_for(int64_t n, int per_thread = 1) {
  int64_t b = (n + (int64_t)kBlock * per_thread - 1) / ((int64_t)kBlock * per_thread);
  if (b < 1) b = 1;
  if (b > 65535ll * 16) b = 65535ll * 16;
  return (int)b;
}

// ---------------------------------------------------------------------------------------------
// relayout: each thread handles a run of consecutive dst positions, seeking its odometer once and
// ticking it after (the SequencerIter walk, furiosa-mapping-types/src/lib.rs:903-946).
// ---------------------------------------------------------------------------------------------
template <typename T, int RUN>
__global__ void __launch_bounds__(kBlock) k_relayout(T* __restrict__ dst, const T* __restrict__ src, int64_t dst_base,
                                                     int64_t src_base, uint32_t count, Wheels<1> w) {
  uint32_t start = (blockIdx.x * (uint32_t)kBlock + threadIdx.x) * RUN;
  uint32_t step = gridDim.x * (uint32_t)kBlock * RUN;
  for (uint32_t p0 = start; p0 < count; p0 += step) {
    uint32_t digit[kMaxWheels];
    int64_t off = 0;
    uint32_t q = p0;
    for (int i = 0; i < w.n; ++i) {
      uint32_t nq = w.div[i].div(q);
      digit[i] = q - nq * w.size[i];
      off += (int64_t)digit[i] * w.stride[0][i];
      q = nq;
    }
    // The run's source offsets are walked first and its reads issued together after a scheduling
    // barrier (a dead or past-the-end position reads element 0, which every non-empty buffer holds,
    // and writes nothing), so a run costs one memory latency rather than one per element.
    int64_t at[RUN];
    bool st[RUN];
#pragma unroll
    for (int r = 0; r < RUN; ++r) {
      const bool in = p0 + r < count;
      bool live = in;
      for (int i = 0; i < w.n; ++i) live &= digit[i] < w.live[i];
      st[r] = live;
      at[r] = live ? src_base + off : 0;
      if (in) {  // tick
        for (int i = 0; i < w.n; ++i) {
          if (digit[i] + 1 < w.size[i]) {
            digit[i] += 1;
            off += w.stride[0][i];
            break;
          }
          off -= (int64_t)digit[i] * w.stride[0][i];
          digit[i] = 0;
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    T v[RUN];
#pragma unroll
    for (int r = 0; r < RUN; ++r) v[r] = src[at[r]];
#pragma unroll
    for (int r = 0; r < RUN; ++r)
      if (st[r]) dst[dst_base + p0 + r] = v[r];
  }
}

// Tiled relayout for a genuine transpose: wheel 0 is contiguous in dst, wheel `j` contiguous in src.
// A 64x64 tile goes through LDS so both the read and the write are coalesced.
template <typename T>
__global__ void __launch_bounds__(256) k_relayout_tiled(T* __restrict__ dst, const T* __restrict__ src,
                                                        int64_t dst_base, int64_t src_base, Wheels<1> w, int jw,
                                                        uint32_t outer_count, uint32_t tiles0, uint32_t tilesj) {
  __shared__ T tile[64][65];
  uint32_t bid = blockIdx.x;
  uint32_t t0 = bid % tiles0;
  bid /= tiles0;
  uint32_t tj = bid % tilesj;
  uint32_t outer = bid / tilesj;
  if (outer >= outer_count) return;
  // Decompose `outer` over the wheels other than 0 and jw; place of each wheel in dst positions.
  int64_t soff = 0, dpos = 0;
  int64_t place = 1;
  int64_t place_j = 0;
  bool live_outer = true;
  uint32_t q = outer;
  for (int i = 0; i < w.n; ++i) {
    if (i == 0) {
      place *= w.size[0];
      continue;
    }
    if (i == jw) {
      place_j = place;
      place *= w.size[i];
      continue;
    }
    uint32_t nq = w.div[i].div(q);
    uint32_t d = q - nq * w.size[i];
    q = nq;
    live_outer &= d < w.live[i];
    soff += (int64_t)d * w.stride[0][i];
    dpos += (int64_t)d * place;
    place *= w.size[i];
  }
  const uint32_t n0 = w.size[0], nj = w.size[jw];
  const int64_t s0 = w.stride[0][0];
  int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;  // 64 x 4
  // read: rows over wheel 0 (dst-contiguous), columns over wheel j (src-contiguous)
  for (int r = ty; r < 64; r += 4) {
    uint32_t d0 = t0 * 64 + r, dj = tj * 64 + tx;
    if (d0 < n0 && dj < nj && live_outer && d0 < w.live[0] && dj < w.live[jw])
      tile[r][tx] = src[src_base + soff + (int64_t)d0 * s0 + dj];
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    uint32_t dj = tj * 64 + r, d0 = t0 * 64 + tx;
    if (d0 < n0 && dj < nj && live_outer && d0 < w.live[0] && dj < w.live[jw])
      dst[dst_base + dpos + (int64_t)dj * place_j + d0] = tile[tx][r];
  }
}

// 16-byte variant of the tiled transpose, for whole 16-byte chunks along both wheel 0 and wheel j
// (sizes, bases and strides multiples of V = 16 / sizeof(T) elements, both wheels fully live):
// src rows are read and dst rows written as 16-byte vectors, the transpose happens in LDS (element
// scatter in, 16-byte reads out).
// TS0 x TSJ tiles (elements along wheel 0 x wheel jw): 64 x 64, or one chunk wide on the side
// whose run is one chunk long, with as many elements as a 64 x 64 tile.
// Wheel bw (if >= 0) is a broadcast axis (src stride 0): the tile is read once and written once
// per live position of it, instead of a block per position re-reading the same source tile.
template <typename T, int TS0, int TSJ>
__global__ void __launch_bounds__(256) k_relayout_tiled16(T* __restrict__ dst, const T* __restrict__ src,
                                                          int64_t dst_base, int64_t src_base, Wheels<1> w, int jw,
                                                          uint32_t outer_count, uint32_t tiles0, uint32_t tilesj,
                                                          int bw) {
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int vec_t;
  constexpr int V = 16 / sizeof(T);  // elements per 16-byte chunk
  constexpr int CPR = TSJ / V;       // chunks per tile row on the read side (along j)
  constexpr int CPW = TS0 / V;       // chunks per tile row on the write side (along d0)
  __shared__ __attribute__((aligned(16))) T tile[TSJ][TS0 + V];  // [j][d0], rows padded by one chunk
  uint32_t bid = blockIdx.x;
  uint32_t t0 = bid % tiles0;
  bid /= tiles0;
  uint32_t tj = bid % tilesj;
  uint32_t outer = bid / tilesj;
  if (outer >= outer_count) return;
  int64_t soff = 0, dpos = 0, place = 1, place_j = 0, place_b = 0;
  bool live_outer = true;
  uint32_t q = outer;
  for (int i = 0; i < w.n; ++i) {
    if (i == 0) {
      place *= w.size[0];
      continue;
    }
    if (i == jw || i == bw) {
      (i == jw ? place_j : place_b) = place;
      place *= w.size[i];
      continue;
    }
    uint32_t nq = w.div[i].div(q);
    uint32_t d = q - nq * w.size[i];
    q = nq;
    live_outer &= d < w.live[i];
    soff += (int64_t)d * w.stride[0][i];
    dpos += (int64_t)d * place;
    place *= w.size[i];
  }
  if (!live_outer) return;  // uniform: a dead outer digit leaves the whole tile unwritten
  const uint32_t n0 = w.size[0], nj = w.size[jw];
  const uint32_t nb = bw >= 0 ? w.live[bw] : 1;
  const int64_t s0 = w.stride[0][0];
  for (int c = threadIdx.x; c < TS0 * CPR; c += 256) {
    const int r = c / CPR, cc = c % CPR;  // src row d0 = r, chunk cc along j
    const uint32_t d0 = t0 * TS0 + r, j0 = tj * TSJ + cc * V;
    if (d0 < n0 && j0 < nj) {
      vec_t v = *(const vec_t*)(src + src_base + soff + (int64_t)d0 * s0 + j0);
      const T* e = (const T*)&v;
#pragma unroll
      for (int k = 0; k < V; ++k) tile[cc * V + k][r] = e[k];
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < TSJ * CPW; c += 256) {
    const int r = c / CPW, cc = c % CPW;  // dst row j = r, chunk cc along d0
    const uint32_t dj = tj * TSJ + r, d0 = t0 * TS0 + cc * V;
    if (dj < nj && d0 < n0) {
      const vec_t v = *(const vec_t*)&tile[r][cc * V];
      T* o = dst + dst_base + dpos + (int64_t)dj * place_j + d0;
      for (uint32_t b = 0; b < nb; ++b) *(vec_t*)(o + (int64_t)b * place_b) = v;
    }
  }
}

// Chunked relayout: the innermost wheel is fully live and contiguous in src (stride 1) and every
// 16-byte chunk of dst positions maps to 16 contiguous, aligned src bytes. One thread moves one
// chunk; only the outer wheels' liveness can drop it.
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int v4i_t;

// Register-tiled relayout for short runs: one thread moves a V x V block (V = elements per
// 16-byte chunk) between wheel 0 (contiguous in dst) and wheel jw (contiguous in src). It reads V
// chunks along jw (one per wheel-0 index), transposes them in registers, and writes V chunks
// along wheel 0 (one per jw index). Consecutive threads take consecutive wheel-0 blocks, then
// jw blocks, so both sides move whole chunks in runs.
template <typename T>
__device__ __forceinline__ void transpose_block(const v4i_t (&in)[16 / sizeof(T)], v4i_t (&out)[16 / sizeof(T)]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int k = 0; k < 4; ++k) out[m][k] = in[k][m];
  } else {
    // 16-bit elements: output chunk m word q = (in[2q] element m, in[2q + 1] element m); element m
    // is the low (m even) or high (m odd) half of word m / 2. v_perm_b32 picks the two halves.
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a = (uint32_t)in[2 * q][m >> 1], b = (uint32_t)in[2 * q + 1][m >> 1];
        out[m][q] = (int)__builtin_amdgcn_perm(b, a, (m & 1) ? 0x07060302u : 0x05040100u);
      }
  }
}

template <typename T>
__global__ void __launch_bounds__(256) k_relayout_rt(T* __restrict__ dst, const T* __restrict__ src, int64_t dst_base,
                                                     int64_t src_base, Wheels<1> w, int jw, uint32_t nb0, uint32_t nbj,
                                                     uint32_t outer_count) {
  constexpr int V = 16 / sizeof(T);
  const uint32_t total = nb0 * nbj * outer_count;
  for (uint32_t idx = blockIdx.x * 256 + threadIdx.x; idx < total; idx += gridDim.x * 256) {
    const uint32_t b0 = idx % nb0, t = idx / nb0, bj = t % nbj, outer = t / nbj;
    int64_t soff = 0, dpos = 0, place = 1, place_j = 0;
    bool live = true;
    uint32_t q = outer;
    for (int i = 0; i < w.n; ++i) {
      if (i == 0) {
        place *= w.size[0];
        continue;
      }
      if (i == jw) {
        place_j = place;
        place *= w.size[i];
        continue;
      }
      const uint32_t nq = w.div[i].div(q);
      const uint32_t d = q - nq * w.size[i];
      q = nq;
      live &= d < w.live[i];
      soff += (int64_t)d * w.stride[0][i];
      dpos += (int64_t)d * place;
      place *= w.size[i];
    }
    if (!live) continue;
    v4i_t in[V], out[V];
    const T* sp = src + src_base + soff + (int64_t)(V * b0) * w.stride[0][0] + V * bj;
#pragma unroll
    for (int k = 0; k < V; ++k) in[k] = *(const v4i_t*)(sp + (int64_t)k * w.stride[0][0]);
    transpose_block<T>(in, out);
    T* dp = dst + dst_base + dpos + (int64_t)(V * bj) * place_j + V * b0;
#pragma unroll
    for (int m = 0; m < V; ++m) *(v4i_t*)(dp + (int64_t)m * place_j) = out[m];
  }
}

template <int VEC>
__global__ void __launch_bounds__(kBlock) k_relayout_chunks(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                            int64_t dst_base_b, int64_t src_base_b, int64_t eb,
                                                            uint32_t nchunks, Wheels<1> w) {
  for (uint32_t c = blockIdx.x * kBlock + threadIdx.x; c < nchunks; c += gridDim.x * kBlock) {
    uint32_t q = c * VEC;
    int64_t off = 0;
    bool live = true;
    for (int i = 0; i < w.n; ++i) {
      uint32_t nq = w.div[i].div(q);
      uint32_t d = q - nq * w.size[i];
      live &= d < w.live[i];
      off += (int64_t)d * w.stride[0][i];
      q = nq;
    }
    if (live)
      *(v4i_t*)(dst + dst_base_b + (int64_t)c * 16) = *(const v4i_t*)(src + src_base_b + off * eb);
  }
}

// The chunked copy of f32 elements whose source is bf16 data standing for its exact widen: each
// four-element chunk reads 8 bytes and writes the widened 16 (bf16_to_f32, the widening cast's rule).
__global__ void __launch_bounds__(kBlock) k_relayout_chunks_widen(float* __restrict__ dst, const uint16_t* __restrict__ src,
                                                                  int64_t dst_base, int64_t src_base, uint32_t nchunks,
                                                                  Wheels<1> w) {
  for (uint32_t c = blockIdx.x * kBlock + threadIdx.x; c < nchunks; c += gridDim.x * kBlock) {
    uint32_t q = c * 4;
    int64_t off = 0;
    bool live = true;
    for (int i = 0; i < w.n; ++i) {
      uint32_t nq = w.div[i].div(q);
      uint32_t d = q - nq * w.size[i];
      live &= d < w.live[i];
      off += (int64_t)d * w.stride[0][i];
      q = nq;
    }
    if (live) {
      const uint2 h = *(const uint2*)(src + src_base + off);
      *(float4*)(dst + dst_base + (int64_t)c * 4) =
          make_float4(bf16_to_f32((uint16_t)h.x), bf16_to_f32((uint16_t)(h.x >> 16)), bf16_to_f32((uint16_t)h.y),
                      bf16_to_f32((uint16_t)(h.y >> 16)));
    }
  }
}

template <typename T>
void relayout_t(hipStream_t s, void* dst, const void* src, int64_t dst_base, int64_t src_base, int64_t count,
                const Wheels<1>& w) {
  // Chunked copy when the innermost dst wheel is src-contiguous and everything is 16-byte aligned.
  // A padded innermost wheel qualifies when its live digits are whole chunks (a window such as
  // `D = 64 # 128`): the kernel skips a chunk with a dead digit, as the element path skips it.
  constexpr int VEC = 16 / sizeof(T);
  if (w.n >= 1 && w.stride[0][0] == 1 && w.live[0] % VEC == 0 && w.size[0] % VEC == 0 && count % VEC == 0 &&
      dst_base % VEC == 0 && src_base % VEC == 0 && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0) {
    bool ok = true;
    for (int i = 1; i < w.n; ++i) ok &= (w.stride[0][i] % VEC) == 0;
    if (ok) {
      int64_t nchunks = count / VEC;
      hipLaunchKernelGGL(k_relayout_chunks<VEC>, dim3(grid_for(nchunks)), dim3(kBlock), 0, s, (uint8_t*)dst,
                         (const uint8_t*)src, dst_base * (int64_t)sizeof(T), src_base * (int64_t)sizeof(T),
                         (int64_t)sizeof(T), (uint32_t)nchunks, w);
      FO_HIP(hipGetLastError());
      return;
    }
  }
  // Tiled transpose when the innermost dst wheel is strided in src and another wheel is the
  // contiguous src run, both big enough to fill a tile, and the positions cover whole wheels.
  // A contiguous src run, or a contiguous dst run, of one 16-byte chunk (e.g. an 8-element packet
  // of bf16) also qualifies, for the 16-byte path only: its tiles are one chunk wide on that side,
  // still coalesced on both.
  int jw = -1;
  bool chunk_run = w.n >= 1 && w.size[0] < 16;  // a one-chunk dst run: the 16-byte path only
  if (w.n >= 2 && w.stride[0][0] != 1 && w.size[0] >= (chunk_run ? VEC : 16) && w.size[0] % (chunk_run ? VEC : 1) == 0) {
    for (int i = 1; i < w.n && jw < 0; ++i)
      if (w.stride[0][i] == 1 && w.size[i] >= 16) jw = i;
    for (int i = 1; i < w.n && jw < 0; ++i)
      if (w.stride[0][i] == 1 && w.size[i] >= VEC && w.size[i] % VEC == 0) {
        jw = i;
        chunk_run = true;
      }
  }
  int64_t total = 1;
  for (int i = 0; i < w.n; ++i) total *= w.size[i];
  // tile shape: one chunk wide on a one-chunk side (TS0 x TSJ = 4096 elements), else 64 x 64
  const int ts0 = chunk_run && w.n >= 1 && w.size[0] < 16 ? VEC : chunk_run ? 4096 / VEC : 64;
  const int tsj = chunk_run && w.n >= 1 && w.size[0] < 16 ? 4096 / VEC : chunk_run ? VEC : 64;
  if (jw > 0 && total == count && chunk_run && (sizeof(T) == 2 || sizeof(T) == 4)) {
    // Short runs on one side: register-tiled V x V blocks, when every chunk is aligned.
    bool rt = w.size[0] % VEC == 0 && w.size[jw] % VEC == 0 && w.live[0] == w.size[0] &&
              w.live[jw] == w.size[jw] && dst_base % VEC == 0 && src_base % VEC == 0 &&
              ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0;
    for (int i = 0; i < w.n && rt; ++i)
      if (i != jw) rt = (w.stride[0][i] % VEC) == 0;
    const uint32_t nb0 = w.size[0] / VEC, nbj = w.size[jw] / VEC;
    const uint32_t outer = (uint32_t)(total / ((int64_t)w.size[0] * w.size[jw]));
    if (rt && (int64_t)nb0 * nbj * outer < (1ll << 31)) {
      hipLaunchKernelGGL(k_relayout_rt<T>, dim3(grid_for((int64_t)nb0 * nbj * outer)), dim3(256), 0, s, (T*)dst,
                         (const T*)src, dst_base, src_base, w, jw, nb0, nbj, outer);
      FO_HIP(hipGetLastError());
      return;
    }
  }
  if (jw > 0 && total == count) {
    uint32_t tiles0 = (w.size[0] + ts0 - 1) / ts0, tilesj = (w.size[jw] + tsj - 1) / tsj;
    uint32_t outer = (uint32_t)(total / ((int64_t)w.size[0] * w.size[jw]));
    // The largest broadcast (src stride 0) outer wheel is looped inside the 16-byte kernel's blocks.
    int bw = -1;
    for (int i = 1; i < w.n; ++i)
      if (i != jw && w.stride[0][i] == 0 && w.size[i] > 1 && (bw < 0 || w.size[i] > w.size[bw])) bw = i;
    const uint32_t outer16 = bw >= 0 ? outer / w.size[bw] : outer;
    const int64_t blocks16 = (int64_t)tiles0 * tilesj * outer16;
    int64_t blocks = (int64_t)tiles0 * tilesj * outer;
    if (blocks < (1ll << 31)) {
      // 16-byte path: whole chunks along both tile axes, every base, stride and place a multiple
      // of a chunk, both tile wheels fully live.
      bool v16 = sizeof(T) >= 2 && w.size[0] % VEC == 0 && w.size[jw] % VEC == 0 && w.live[0] == w.size[0] &&
                 w.live[jw] == w.size[jw] && dst_base % VEC == 0 && src_base % VEC == 0 &&
                 ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 16) == 0;
      for (int i = 0; i < w.n && v16; ++i)
        if (i != jw) v16 = (w.stride[0][i] % VEC) == 0;
      if (v16 || !chunk_run) {
        if (v16 && ts0 == VEC)
          hipLaunchKernelGGL((k_relayout_tiled16<T, VEC, 4096 / VEC>), dim3((uint32_t)blocks16), dim3(256), 0, s,
                             (T*)dst, (const T*)src, dst_base, src_base, w, jw, outer16, tiles0, tilesj, bw);
        else if (v16 && tsj == VEC)
          hipLaunchKernelGGL((k_relayout_tiled16<T, 4096 / VEC, VEC>), dim3((uint32_t)blocks16), dim3(256), 0, s,
                             (T*)dst, (const T*)src, dst_base, src_base, w, jw, outer16, tiles0, tilesj, bw);
        else if (v16)
          hipLaunchKernelGGL((k_relayout_tiled16<T, 64, 64>), dim3((uint32_t)blocks16), dim3(256), 0, s, (T*)dst,
                             (const T*)src, dst_base, src_base, w, jw, outer16, tiles0, tilesj, bw);
        else
          hipLaunchKernelGGL(k_relayout_tiled<T>, dim3((uint32_t)blocks), dim3(256), 0, s, (T*)dst, (const T*)src,
                             dst_base, src_base, w, jw, outer, tiles0, tilesj);
        FO_HIP(hipGetLastError());
        return;
      }
    }
  }
  constexpr int RUN = 8;
  hipLaunchKernelGGL((k_relayout<T, RUN>), dim3(grid_for(count, RUN)), dim3(kBlock), 0, s, (T*)dst, (const T*)src,
                     dst_base, src_base, (uint32_t)count, w);
  FO_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------
// Relayout chain (lazy relayout fusion): each final position walks back through the steps. A
// position a step did not write reads as the zero of its fresh storage (Tensor::transpose zeroes
// its destination, tensor/mod.rs:302-306); one the last step does not write is left alone.
// ---------------------------------------------------------------------------------------------
// Walks final position `pos` (< c.total) back through the steps: 0 = read src at *pos, 1 = zero,
// 2 = not written.
__device__ __forceinline__ int chain_walk(const Chain& c, int64_t* pos_io) {
  const int unwritten = c.zero_unwritten ? 1 : 2;
  int64_t pos = *pos_io;
  for (int k = c.n - 1; k >= 0; --k) {
    const ChainStep& st = c.step[k];
    if (pos >= (int64_t)st.count) return k == c.n - 1 ? unwritten : 1;
    uint32_t q = (uint32_t)pos;
    int64_t off = 0;
    bool live = true;
    for (int i = 0; i < st.w.n; ++i) {
      const uint32_t nq = st.w.div[i].div(q);
      const uint32_t d = q - nq * st.w.size[i];
      live &= d < st.w.live[i];
      off += (int64_t)d * st.w.stride[0][i];
      q = nq;
    }
    if (!live) return k == c.n - 1 ? unwritten : 1;
    pos = st.src_base + off;
  }
  *pos_io = pos;
  return 0;
}

template <typename T>
__global__ void __launch_bounds__(kBlock) k_relayout_chain(T* __restrict__ dst, const T* __restrict__ src, Chain c) {
  for (uint32_t p = blockIdx.x * kBlock + threadIdx.x; p < c.total; p += gridDim.x * kBlock) {
    int64_t pos = p;
    const int state = chain_walk(c, &pos);
    if (state == 0)
      dst[p] = src[pos];
    else if (state == 1)
      dst[p] = T(0);
  }
}

// The same walk over 4-bit elements (two per byte, element 2k in the low nibble of byte k; the
// reference packs sub-byte storage this way, storage/buf.rs:56-80, scalar.rs:1093-1117). Final
// position p is element dst_base + p of dst. One thread owns one dst byte and writes it whole, so
// the byte's other nibble -- outside the window, or not written -- keeps what dst holds.
__global__ void __launch_bounds__(kBlock) k_relayout_chain_nibble(uint8_t* __restrict__ dst,
                                                                  const uint8_t* __restrict__ src, Chain c,
                                                                  uint64_t dst_base) {
  const uint64_t b0 = dst_base / 2, nbytes = (dst_base + c.total + 1) / 2 - b0;
  for (uint64_t t = blockIdx.x * (uint64_t)kBlock + threadIdx.x; t < nbytes; t += (uint64_t)gridDim.x * kBlock) {
    const uint64_t b = b0 + t;
    uint32_t byte = dst[b];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t p = (int64_t)(2 * b + h) - (int64_t)dst_base;
      if (p < 0 || p >= (int64_t)c.total) continue;
      int64_t pos = p;
      const int state = chain_walk(c, &pos);
      if (state == 2) continue;
      const uint32_t v = state == 0 ? (src[pos >> 1] >> (4 * (pos & 1))) & 0xfu : 0u;
      byte = (byte & ~(0xfu << (4 * h))) | (v << (4 * h));
    }
    dst[b] = (uint8_t)byte;
  }
}

// ---------------------------------------------------------------------------------------------
// transmute: dst live rank k <- src live rank k (place_live_elems, storage/buf.rs:785-797).
// `ds` walks dst wire positions (size = extent, live = count); `ss` maps a live rank to a src
// wire position (size = live count, stride = wire place).
// ---------------------------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kBlock) k_transmute(T* __restrict__ dst, const T* __restrict__ src, uint32_t count,
                                                      Wheels<1> ds, Wheels<1> ss) {
  for (uint32_t p = blockIdx.x * kBlock + threadIdx.x; p < count; p += gridDim.x * kBlock) {
    uint32_t q = p;
    bool live = true;
    uint32_t rank = 0, rplace = 1;
    for (int i = 0; i < ds.n; ++i) {
      uint32_t nq = ds.div[i].div(q);
      uint32_t d = q - nq * ds.size[i];
      q = nq;
      live &= d < ds.live[i];
      rank += d * rplace;
      rplace *= ds.live[i];
    }
    if (!live) {
      dst[p] = T(0);
      continue;
    }
    int64_t off = 0;
    uint32_t r = rank;
    for (int i = 0; i < ss.n; ++i) {
      uint32_t nr = ss.div[i].div(r);
      off += (int64_t)(r - nr * ss.size[i]) * ss.stride[0][i];
      r = nr;
    }
    dst[p] = src[off];
  }
}

// ---------------------------------------------------------------------------------------------
// scatter / gather (storage/buf.rs:485-576). Both walk a stream of (payload position, slot): the
// src and dst offsets come from two wheel lists, and the slot's index picks the position on the
// indexed axis. An index that is negative or past the axis is skipped and raises `flag` (the
// reference panics there); the host reports it.
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int64_t wheel_offset(const Wheels<1>& w, uint32_t q) {
  int64_t off = 0;
  for (int i = 0; i < w.n; ++i) {
    uint32_t nq = w.div[i].div(q);
    off += (int64_t)(q - nq * w.size[i]) * w.stride[0][i];
    q = nq;
  }
  return off;
}

// Decoded index (decode_indices, buf.rs:801-812) or -1 when it is out of range.
__device__ __forceinline__ int32_t decode_index(const int32_t* __restrict__ idx, uint32_t i, int32_t div,
                                                uint32_t axis_size) {
  int32_t raw = idx[i];
  if (raw < 0) return -1;
  int32_t a = raw / div;
  return (uint32_t)a < axis_size ? a : -1;
}

// dst[off_d(p, r)] = src[off_s(p, index[r])] for every payload position p and index slot r.
template <typename T>
__global__ void __launch_bounds__(kBlock) k_gather(T* __restrict__ dst, const T* __restrict__ src,
                                                   const int32_t* __restrict__ idx, uint32_t total, FastDiv rdiv,
                                                   uint32_t axis_size, int32_t div, Wheels<1> ws, Wheels<1> wd,
                                                   int32_t* __restrict__ flag) {
  for (uint32_t t = blockIdx.x * kBlock + threadIdx.x; t < total; t += gridDim.x * kBlock) {
    uint32_t p = rdiv.div(t), r = t - p * rdiv.d;
    int32_t a = decode_index(idx, r, div, axis_size);
    if (a < 0) {
      *flag = 1;
      continue;
    }
    dst[wheel_offset(wd, t)] = src[wheel_offset(ws, p * axis_size + (uint32_t)a)];
  }
}

// 16-byte form: the innermost payload wheel is contiguous in both memories and a whole number of
// V-element chunks, so payload positions c*V .. c*V+V-1 are adjacent on both sides. Thread (r, c)
// moves chunk c of slot r; consecutive threads take consecutive chunks of one row.
// The scatter's threads move kChunkRuns chunks a grid stride apart, each chunk's data read issued
// with its index read (it does not depend on it), the winner checks and writes after all of them
// (measured 21.6 -> 21.0 us for 131072 rows of 256 bytes; the same for the gather, whose data read
// waits for the index, measured 22.6 -> 27.0 us and is not used).
constexpr int kChunkRuns = 4;
template <int V>
__global__ void __launch_bounds__(kBlock) k_gather_vec(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                       int64_t eb, const int32_t* __restrict__ idx, uint32_t total,
                                                       FastDiv cdiv, uint32_t slots, uint32_t axis_size, int32_t div,
                                                       Wheels<1> ws, Wheels<1> wd, int32_t* __restrict__ flag) {
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int vec_t;
  for (uint32_t t = blockIdx.x * kBlock + threadIdx.x; t < total; t += gridDim.x * kBlock) {
    uint32_t r = cdiv.div(t), c = t - r * cdiv.d;
    int32_t a = decode_index(idx, r, div, axis_size);
    if (a < 0) {
      *flag = 1;
      continue;
    }
    const uint32_t p = c * V;
    *(vec_t*)(dst + wheel_offset(wd, p * slots + r) * eb) =
        *(const vec_t*)(src + wheel_offset(ws, p * axis_size + (uint32_t)a) * eb);
  }
}

template <int V>
__global__ void __launch_bounds__(kBlock) k_scatter_vec(uint8_t* __restrict__ dst, const uint8_t* __restrict__ src,
                                                        int64_t eb, const int32_t* __restrict__ idx,
                                                        const uint64_t* __restrict__ win, uint64_t tag, uint32_t total,
                                                        FastDiv cdiv, uint32_t keys, uint32_t axis_size, int32_t div,
                                                        Wheels<1> ws, Wheels<1> wd, int32_t* __restrict__ flag) {
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int vec_t;
  constexpr int U = kChunkRuns;  // as in k_gather_vec; the data read does not wait for the index
  const uint64_t stride = (uint64_t)gridDim.x * kBlock;
  for (uint64_t t0 = (uint64_t)blockIdx.x * kBlock + threadIdx.x; t0 < total; t0 += U * stride) {
    uint32_t k[U], c[U];
    int32_t a[U];
    vec_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t t = t0 + u * stride;
      const uint32_t tt = t < total ? (uint32_t)t : 0u;
      k[u] = cdiv.div(tt);
      c[u] = tt - k[u] * cdiv.d;
      a[u] = t < total ? decode_index(idx, k[u], div, axis_size) : -1;
      if (t < total) v[u] = *(const vec_t*)(src + wheel_offset(ws, c[u] * V * keys + k[u]) * eb);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (a[u] >= 0 && (!win || win[a[u]] == (tag | k[u])))
        *(vec_t*)(dst + wheel_offset(wd, c[u] * V * axis_size + (uint32_t)a[u]) * eb) = v[u];
      else if (!win && a[u] < 0 && t0 + u * stride < total)
        *flag = 1;  // no winners pass ran to report it
    }
  }
}

// Whether payload positions come in adjacent 16-byte runs on both sides: the innermost payload
// wheel (part 0) has stride 1 and a multiple of V digits, every other stride is a multiple of V.
bool payload_vec_ok(const Wheels<1>& w, int inner_slot_wheels, int V) {
  if (inner_slot_wheels >= w.n) return false;
  const int i0 = inner_slot_wheels;  // wheels are innermost-first: slot / axis wheels come first
  if (w.stride[0][i0] != 1 || w.size[i0] % V != 0 || w.live[i0] != w.size[i0]) return false;
  for (int i = 0; i < w.n; ++i)
    if (i != i0 && w.stride[0][i] % V != 0) return false;
  return true;
}

// win[a] = tag | the last key slot whose index is a: the serial scatter's last write wins. `tag` is
// the call's generation in the high word, so entries of earlier calls (lower generations) lose to
// any key of this one and the array never needs clearing between calls.
__global__ void __launch_bounds__(kBlock) k_scatter_winners(const int32_t* __restrict__ idx, uint32_t keys,
                                                            uint32_t axis_size, int32_t div, uint64_t* __restrict__ win,
                                                            uint64_t tag, int32_t* __restrict__ flag) {
  for (uint32_t k = blockIdx.x * kBlock + threadIdx.x; k < keys; k += gridDim.x * kBlock) {
    int32_t a = decode_index(idx, k, div, axis_size);
    if (a < 0)
      *flag = 1;
    else
      atomicMax((unsigned long long*)(win + a), (unsigned long long)(tag | k));
  }
}

// dst[off_d(p, index[k])] = src[off_s(p, k)] for the winning key slot k of each target.
template <typename T>
__global__ void __launch_bounds__(kBlock) k_scatter(T* __restrict__ dst, const T* __restrict__ src,
                                                    const int32_t* __restrict__ idx, const uint64_t* __restrict__ win,
                                                    uint64_t tag, uint32_t total, FastDiv kdiv, uint32_t axis_size,
                                                    int32_t div, Wheels<1> ws, Wheels<1> wd, int32_t* __restrict__ flag) {
  for (uint32_t t = blockIdx.x * kBlock + threadIdx.x; t < total; t += gridDim.x * kBlock) {
    uint32_t p = kdiv.div(t), k = t - p * kdiv.d;
    int32_t a = decode_index(idx, k, div, axis_size);
    if (a < 0) {
      if (!win) *flag = 1;  // no winners pass ran to report it
      continue;
    }
    if (win && win[a] != (tag | k)) continue;
    dst[wheel_offset(wd, p * axis_size + (uint32_t)a)] = src[wheel_offset(ws, t)];
  }
}

}  // namespace

void launch_relayout_chain_nibble(hipStream_t s, void* dst, const void* src, const Chain& c, uint64_t dst_base) {
  const int64_t nbytes = (int64_t)((dst_base + c.total + 1) / 2 - dst_base / 2);
  hipLaunchKernelGGL(k_relayout_chain_nibble, dim3(grid_for(nbytes)), dim3(kBlock), 0, s, (uint8_t*)dst,
                     (const uint8_t*)src, c, dst_base);
  FO_HIP(hipGetLastError());
}

void launch_relayout_chain(hipStream_t s, void* dst, const void* src, int64_t elem_bytes, const Chain& c) {
  dim3 g(grid_for((int64_t)c.total)), b(kBlock);
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(k_relayout_chain<uint8_t>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, c);
      break;
    case 2:
      hipLaunchKernelGGL(k_relayout_chain<uint16_t>, g, b, 0, s, (uint16_t*)dst, (const uint16_t*)src, c);
      break;
    default:
      hipLaunchKernelGGL(k_relayout_chain<uint32_t>, g, b, 0, s, (uint32_t*)dst, (const uint32_t*)src, c);
  }
  FO_HIP(hipGetLastError());
}

void launch_relayout(hipStream_t s, void* dst, const void* src, int64_t eb, int64_t dst_base, int64_t src_base,
                     int64_t count, const Wheels<1>& w) {
  switch (eb) {
    case 1:
      return relayout_t<uint8_t>(s, dst, src, dst_base, src_base, count, w);
    case 2:
      return relayout_t<uint16_t>(s, dst, src, dst_base, src_base, count, w);
    case 4:
      return relayout_t<uint32_t>(s, dst, src, dst_base, src_base, count, w);
  }
  throw InvalidArg("relayout: unsupported element size");
}

bool launch_relayout_widen(hipStream_t s, float* dst, const uint16_t* src, int64_t dst_base, int64_t src_base,
                           int64_t count, const Wheels<1>& w) {
  // The f32 chunked copy's conditions, with the source 8-byte aligned (its chunks are 4 bf16).
  if (!(w.n >= 1 && w.stride[0][0] == 1 && w.live[0] % 4 == 0 && w.size[0] % 4 == 0 && count % 4 == 0 &&
        dst_base % 4 == 0 && src_base % 4 == 0 && ((uintptr_t)dst % 16) == 0 && ((uintptr_t)src % 8) == 0))
    return false;
  for (int i = 1; i < w.n; ++i)
    if (w.stride[0][i] % 4 != 0) return false;
  const int64_t nchunks = count / 4;
  hipLaunchKernelGGL(k_relayout_chunks_widen, dim3(grid_for(nchunks)), dim3(kBlock), 0, s, dst, src, dst_base, src_base,
                     (uint32_t)nchunks, w);
  FO_HIP(hipGetLastError());
  return true;
}

void launch_transmute(hipStream_t s, void* dst, const void* src, int64_t eb, int64_t dst_count,
                      const Wheels<1>& dst_self, const Wheels<1>& src_self) {
  dim3 g(grid_for(dst_count)), b(kBlock);
  switch (eb) {
    case 1:
      hipLaunchKernelGGL(k_transmute<uint8_t>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, (uint32_t)dst_count,
                         dst_self, src_self);
      break;
    case 2:
      hipLaunchKernelGGL(k_transmute<uint16_t>, g, b, 0, s, (uint16_t*)dst, (const uint16_t*)src,
                         (uint32_t)dst_count, dst_self, src_self);
      break;
    case 4:
      hipLaunchKernelGGL(k_transmute<uint32_t>, g, b, 0, s, (uint32_t*)dst, (const uint32_t*)src,
                         (uint32_t)dst_count, dst_self, src_self);
      break;
    default:
      throw InvalidArg("transmute: unsupported element size");
  }
  FO_HIP(hipGetLastError());
}

// ---------------------------------------------------------------------------------------------
// reduce: one thread per output cell, folding the live residue in wire order -- the exact fold
// order of BufStorage::reduce (buf.rs:360-373), so f32 results are bit-identical to the emulator.
// When there are too few output cells to fill the GPU, a wave per cell folds strided slices and
// combines them (exact for integer ops; reassociated for floats, like the emulator's own caveat
// at buf.rs:316-330).
// ---------------------------------------------------------------------------------------------
namespace {

template <typename T>
struct RedT;
template <>
struct RedT<float> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return ((const float*)p)[i]; }
  static __device__ __forceinline__ void store(void* p, int64_t i, float v) { ((float*)p)[i] = v; }
  static __device__ __forceinline__ float from_bits(uint32_t b) { return bits_f32(b); }
  static __device__ __forceinline__ float apply(int op, float a, float b) {
    switch (op) {
      case FO_RED_ADD:
        return __fadd_rn(a, b);
      case FO_RED_MAX:
        return fmaxf(a, b);
      case FO_RED_MIN:
        return fminf(a, b);
      default:
        return __fmul_rn(a, b);
    }
  }
};
// An f32 fold over bf16 data standing for its exact widen (a deferred widening cast): each element
// is widened on load by the cast's own rule, then folded as f32.
struct WidenedBf16 {};
template <>
struct RedT<WidenedBf16> : RedT<float> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) { return bf16_to_f32(((const uint16_t*)p)[i]); }
};
// An f32 fold over f32 data standing for the widen of its bf16 narrow (a deferred narrow read
// through a deferred widen): each element is rounded on load by the narrow's rule, then widened.
struct RoundedBf16 {};
template <>
struct RedT<RoundedBf16> : RedT<float> {
  static __device__ __forceinline__ float load(const void* p, int64_t i) {
    return bf16_to_f32(f32_to_bf16(((const float*)p)[i]));
  }
};

template <>
struct RedT<int32_t> {
  static __device__ __forceinline__ int32_t load(const void* p, int64_t i) { return ((const int32_t*)p)[i]; }
  static __device__ __forceinline__ void store(void* p, int64_t i, int32_t v) { ((int32_t*)p)[i] = v; }
  static __device__ __forceinline__ int32_t from_bits(uint32_t b) { return (int32_t)b; }
  static __device__ __forceinline__ int32_t apply(int op, int32_t a, int32_t b) {
    switch (op) {
      case FO_RED_ADD:
        return (int32_t)((uint32_t)a + (uint32_t)b);
      case FO_RED_MAX:
        return a > b ? a : b;
      case FO_RED_MIN:
        return a < b ? a : b;
      case FO_RED_MUL:
        return (int32_t)((uint32_t)a * (uint32_t)b);
      default: {
        int64_t r = (int64_t)a + b;
        return (int32_t)(r > INT32_MAX ? INT32_MAX : r < INT32_MIN ? INT32_MIN : r);
      }
    }
  }
};
// bf16 folds use `half` arithmetic: each step widens exactly and rounds back (no flush).
struct Bf16Red {};
template <>
struct RedT<Bf16Red> {
  static __device__ __forceinline__ uint16_t load(const void* p, int64_t i) { return ((const uint16_t*)p)[i]; }
  static __device__ __forceinline__ void store(void* p, int64_t i, uint16_t v) { ((uint16_t*)p)[i] = v; }
  static __device__ __forceinline__ uint16_t from_bits(uint32_t b) { return (uint16_t)b; }
  static __device__ __forceinline__ uint16_t apply(int op, uint16_t a, uint16_t b) {
    float fa = half_bf16_to_f32(a), fb = half_bf16_to_f32(b);
    switch (op) {
      case FO_RED_ADD:
        return half_round_bf16(__fadd_rn(fa, fb));
      case FO_RED_MAX:  // half's Ord-free max: f32::max semantics on the widened values
        return half_round_bf16(fmaxf(fa, fb));
      case FO_RED_MIN:
        return half_round_bf16(fminf(fa, fb));
      default:
        return half_round_bf16(__fmul_rn(fa, fb));
    }
  }
};

// Residue reads batched per fold step (see k_reduce_thread / k_contract_generic).
constexpr int kBatch = 16;

// One tick of an odometer over wheels w (innermost first): the digits and the offsets into each
// of the NMEM memories advance to the next position.
// The digits are indexed by a runtime wheel count, so they may live in indexed registers; an
// indexed register access makes the compiler wait for every load in flight. Batched readers
// therefore compute a batch's offsets first and issue its loads after a scheduling barrier.
template <int NMEM>
__device__ __forceinline__ void odometer_step(const Wheels<NMEM>& w, uint32_t (&digit)[kMaxWheels],
                                              int64_t (&off)[NMEM]) {
  for (int i = 0; i < w.n; ++i) {
    if (digit[i] + 1 < w.size[i]) {
      digit[i]++;
#pragma unroll
      for (int k = 0; k < NMEM; ++k) off[k] += w.stride[k][i];
      return;
    }
#pragma unroll
    for (int k = 0; k < NMEM; ++k) off[k] -= (int64_t)digit[i] * w.stride[k][i];
    digit[i] = 0;
  }
}

// The odometer at stream position pos: digits and the offsets added to `off`.
template <int NMEM>
__device__ __forceinline__ void odometer_seek(const Wheels<NMEM>& w, uint32_t pos, uint32_t (&digit)[kMaxWheels],
                                              int64_t (&off)[NMEM]) {
  for (int i = 0; i < kMaxWheels; ++i) digit[i] = 0;
  uint32_t q = pos;
  for (int i = 0; i < w.n; ++i) {
    const uint32_t nq = w.div[i].div(q);
    digit[i] = q - nq * w.size[i];
#pragma unroll
    for (int k = 0; k < NMEM; ++k) off[k] += (int64_t)digit[i] * w.stride[k][i];
    q = nq;
  }
}

// Lane `lane`'s 64-bit value, for every lane (`lane` a compile-time constant).
__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Wire offsets of output cell o (decoded from the out wheels) into each memory; dead when a digit
// is padding (or o is past the output).
template <int NMEM>
__device__ __forceinline__ bool cell_base(const Wheels<NMEM>& ow, uint32_t o, uint32_t count, int64_t (&b)[NMEM]) {
  bool dead = o >= count;
#pragma unroll
  for (int k = 0; k < NMEM; ++k) b[k] = 0;
  uint32_t q = dead ? 0 : o;
  for (int i = 0; i < ow.n; ++i) {
    const uint32_t nq = ow.div[i].div(q);
    const uint32_t d = q - nq * ow.size[i];
    dead |= d >= ow.live[i];
#pragma unroll
    for (int k = 0; k < NMEM; ++k) b[k] += (int64_t)d * ow.stride[k][i];
    q = nq;
  }
  return dead;
}

template <typename Tag>
__global__ void __launch_bounds__(kBlock) k_reduce_thread(void* dst, const void* src, int64_t src_len,
                                                          uint32_t out_count, Wheels<1> ow, Wheels<1> rw, int op,
                                                          uint32_t identity) {
  using R = RedT<Tag>;
  for (uint32_t o = blockIdx.x * kBlock + threadIdx.x; o < out_count; o += gridDim.x * kBlock) {
    int64_t base = 0;
    uint32_t q = o;
    bool dead = false;
    for (int i = 0; i < ow.n; ++i) {
      uint32_t nq = ow.div[i].div(q);
      const uint32_t d = q - nq * ow.size[i];
      dead |= d >= ow.live[i];
      base += (int64_t)d * ow.stride[0][i];
      q = nq;
    }
    auto acc = R::from_bits(identity);
    if (dead) {  // a padding cell has no reads and keeps the identity (buf.rs:355-368)
      R::store(dst, o, acc);
      continue;
    }
    uint32_t digit[kMaxWheels] = {};
    int64_t off[1] = {base};
    uint32_t total = 1;
    for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
    // kBatch reads are issued before they are folded (still in wire order), so a long residue is
    // not one memory latency per element.
    for (uint32_t r0 = 0; r0 < total; r0 += kBatch) {
      decltype(R::load(src, 0)) v[kBatch];
      bool ok[kBatch];
      int64_t at[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const bool in = r0 + u < total;
        ok[u] = in && off[0] >= 0 && off[0] < src_len;
        at[u] = ok[u] ? off[0] : 0;
        if (in) odometer_step(rw, digit, off);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = R::load(src, at[u]);  // all reads in flight together
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (ok[u]) acc = R::apply(op, acc, v[u]);
    }
    R::store(dst, o, acc);
  }
}

// Thread per cell over a residue of one wheel (`total` elements `rstride` apart): the reads of a
// batch are issued together and folded in order, the emulator's serial fold.
template <typename Tag>
__global__ void __launch_bounds__(kBlock) k_reduce_strided(void* dst, const void* src, int64_t src_len,
                                                           uint32_t out_count, Wheels<1> ow, uint32_t total,
                                                           int64_t rstride, int op, uint32_t identity) {
  using R = RedT<Tag>;
  constexpr int U = 16;
  for (uint32_t o = blockIdx.x * kBlock + threadIdx.x; o < out_count; o += gridDim.x * kBlock) {
    int64_t b[1];
    const bool dead = cell_base(ow, o, out_count, b);
    auto acc = R::from_bits(identity);
    if (!dead) {
      for (uint32_t r0 = 0; r0 < total; r0 += U) {
        decltype(R::load(src, 0)) v[U];
        bool ok[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t off = b[0] + (int64_t)(r0 + u) * rstride;
          ok[u] = r0 + u < total && off >= 0 && off < src_len;
          v[u] = R::load(src, ok[u] ? off : 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (ok[u]) acc = R::apply(op, acc, v[u]);
      }
    }
    R::store(dst, o, acc);
  }
}

template <typename Tag>
__global__ void __launch_bounds__(kBlock) k_reduce_wave(void* dst, const void* src, int64_t src_len, uint32_t out_count,
                                                        Wheels<1> ow, Wheels<1> rw, int op, uint32_t identity,
                                                        uint32_t neutral) {
  using R = RedT<Tag>;
  const int lane = threadIdx.x & 63;
  uint32_t wave = (blockIdx.x * kBlock + threadIdx.x) >> 6;
  uint32_t nwaves = (gridDim.x * kBlock) >> 6;
  uint32_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  for (uint32_t o = wave; o < out_count; o += nwaves) {
    int64_t base = 0;
    uint32_t q = o;
    bool dead = false;
    for (int i = 0; i < ow.n; ++i) {
      uint32_t nq = ow.div[i].div(q);
      const uint32_t d = q - nq * ow.size[i];
      dead |= d >= ow.live[i];
      base += (int64_t)d * ow.stride[0][i];
      q = nq;
    }
    // Each lane folds its strided slice from the op's neutral element, so the caller's identity
    // enters the result exactly once, after the lanes combine.
    auto acc = R::from_bits(neutral);
    if (rw.n == 1 && rw.stride[0][0] == 1) {
      // One contiguous residue run: 8 coalesced reads per lane in flight, no odometer.
      const int64_t lim = dead ? 0 : min((int64_t)total, src_len - base);
      int64_t r = lane;
      for (; r + 7 * 64 < lim; r += 8 * 64) {
        decltype(R::load(src, 0)) v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = R::load(src, base + r + 64 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = R::apply(op, acc, v[u]);
      }
      for (; r < lim; r += 64) acc = R::apply(op, acc, R::load(src, base + r));
    } else {
      for (uint32_t r = lane; r < total && !dead; r += 64) {
        int64_t off = base;
        uint32_t rr = r;
        for (int i = 0; i < rw.n; ++i) {
          uint32_t nr = rw.div[i].div(rr);
          off += (int64_t)(rr - nr * rw.size[i]) * rw.stride[0][i];
          rr = nr;
        }
        if (off >= 0 && off < src_len) acc = R::apply(op, acc, R::load(src, off));
      }
    }
    for (int m = 32; m >= 1; m >>= 1) {
      auto other = __shfl_xor(acc, m, 64);
      acc = R::apply(op, acc, other);
    }
    if (lane == 0) R::store(dst, o, dead ? R::from_bits(identity) : R::apply(op, R::from_bits(identity), acc));
  }
}

// BufStorage::reduce's per-cell fold with coalesced reads, organised as k_contract_tiled: one wave
// per 64 output cells, 64 residue positions at a time read by consecutive lanes and staged in LDS,
// then folded per cell in residue order from the identity.
template <typename Tag>
__global__ void __launch_bounds__(256) k_reduce_tiled(void* dst, const void* __restrict__ src, int64_t src_len,
                                                      uint32_t out_count, Wheels<1> ow, Wheels<1> rw, int op,
                                                      uint32_t identity, uint32_t total) {
  using R = RedT<Tag>;
  using V = decltype(R::load(src, 0));
  __shared__ V vals[4][64][65];
  __shared__ uint64_t valid[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (uint64_t g0 = ((uint64_t)blockIdx.x * 4 + wave) * 64; g0 < out_count; g0 += (uint64_t)gridDim.x * 256) {
    const uint32_t o = (uint32_t)g0 + lane;
    int64_t b[1];
    const bool dead = cell_base(ow, o, out_count, b);
    auto acc = R::from_bits(identity);
    for (uint32_t r0 = 0; r0 < total; r0 += 64) {
      const bool rin = r0 + lane < total;
      int64_t d = 0;
      if (rin) {
        uint32_t q = r0 + lane;
        for (int i = 0; i < rw.n; ++i) {
          const uint32_t nq = rw.div[i].div(q);
          d += (int64_t)(q - nq * rw.size[i]) * rw.stride[0][i];
          q = nq;
        }
      }
#pragma unroll
      for (int cg = 0; cg < 64; cg += 16) {
        V v[16];
        bool ok[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int64_t a = readlane64(b[0], cg + u) + d;
          ok[u] = rin && a >= 0 && a < src_len;
          v[u] = R::load(src, ok[u] ? a : 0);
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          vals[wave][cg + u][lane] = v[u];
          const uint64_t mask = __ballot(ok[u]);
          if (lane == 0) valid[wave][cg + u] = mask;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint64_t vm = valid[wave][lane];
      const int cnt = (int)min(64u, total - r0);
      if (!dead)
        for (int j = 0; j < cnt; ++j)
          if ((vm >> j) & 1u) acc = R::apply(op, acc, vals[wave][lane][j]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (o < out_count) R::store(dst, o, acc);
  }
}

// Reduce with the residue split into kSeg segments per cell: block = 64 consecutive output cells
// (lanes; consecutive cells sit at consecutive addresses when the out wheel is contiguous) x kSeg
// waves, each folding its segment of the residue from the op's neutral element, kBatch reads in
// flight per step; the segments then combine in order through LDS, and the caller's identity enters
// once. A regrouping: exact for the integer ops, reassociated for f32.
constexpr int kSeg = 16;
template <typename Tag>
__global__ void __launch_bounds__(64 * kSeg) k_reduce_cols(void* dst, const void* __restrict__ src, int64_t src_len,
                                                           uint32_t out_count, Wheels<1> ow, Wheels<1> rw, int op,
                                                           uint32_t identity, uint32_t neutral, uint32_t total) {
  using R = RedT<Tag>;
  using V = decltype(R::load(src, 0));
  __shared__ V part[kSeg][64];
  const int seg = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t o = blockIdx.x * 64 + lane;
  int64_t b[1];
  const bool dead = cell_base(ow, o, out_count, b);
  auto acc = R::from_bits(neutral);
  const uint32_t len = (total + kSeg - 1) / kSeg;
  const uint32_t r_begin = min(total, (uint32_t)seg * len), r_end = min(total, r_begin + len);
  if (!dead && r_begin < r_end) {
    // the odometer at r_begin
    uint32_t digit[kMaxWheels];
    int64_t off[1] = {b[0]};
    odometer_seek(rw, r_begin, digit, off);
    for (uint32_t r0 = r_begin; r0 < r_end; r0 += kBatch) {
      V v[kBatch];
      bool ok[kBatch];
      int64_t at[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const bool in = r0 + u < r_end;
        ok[u] = in && off[0] >= 0 && off[0] < src_len;
        at[u] = ok[u] ? off[0] : 0;
        if (in) odometer_step(rw, digit, off);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) v[u] = R::load(src, at[u]);  // all reads in flight together
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (ok[u]) acc = R::apply(op, acc, v[u]);
    }
  }
  part[seg][lane] = acc;
  __syncthreads();
  if (seg == 0 && o < out_count) {
    auto total_acc = R::from_bits(identity);
    if (!dead)
      for (int k = 0; k < kSeg; ++k) total_acc = R::apply(op, total_acc, part[k][lane]);
    R::store(dst, o, total_acc);
  }
}

// The same fold for contiguous output cells split over many residue chunks (two passes): pass one
// folds chunk c of the residue for 256 cells per block -- each lane four adjacent cells through
// 16-byte loads, so a wave reads 1 KiB per residue step, the block's four waves splitting the chunk
// and combining in wave order -- into partials[c][cell]; pass two folds each cell's partials in
// chunk order, from the caller's identity. 4-byte folds that may be regrouped only (f32, and the
// integer ops except the saturating add); the host checks the layout (cells in whole groups of
// four, 16-byte aligned offsets, every read inside the source).
template <typename Tag>
struct Vec4T;
template <>
struct Vec4T<float> {
  typedef float type __attribute__((ext_vector_type(4)));
};
template <>
struct Vec4T<int32_t> {
  typedef int type __attribute__((ext_vector_type(4)));
};

// The rows [r_begin, r_end) of one 4-column group folded into acc, 16 rows' loads in flight.
template <typename Tag, int OP>
__device__ __forceinline__ typename Vec4T<Tag>::type cols4_rows(const void* __restrict__ src, const Wheels<1>& rw,
                                                               int64_t base, uint32_t r_begin, uint32_t r_end,
                                                               typename Vec4T<Tag>::type acc) {
  using R = RedT<Tag>;
  using V4 = typename Vec4T<Tag>::type;
  constexpr int U = 16;
  uint32_t digit[kMaxWheels];
  int64_t off[1] = {base};
  odometer_seek(rw, r_begin, digit, off);
  const V4* s4 = (const V4*)src;
  uint32_t r = r_begin;
  for (; r + U <= r_end; r += U) {
    V4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      v[u] = __builtin_nontemporal_load(s4 + (off[0] >> 2));
      odometer_step(rw, digit, off);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = R::apply(OP, acc[e], v[u][e]);
  }
  for (; r < r_end; ++r) {
    const V4 v = __builtin_nontemporal_load(s4 + (off[0] >> 2));
    odometer_step(rw, digit, off);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = R::apply(OP, acc[e], v[e]);
  }
  return acc;
}

template <typename Tag>
__global__ void __launch_bounds__(256) k_reduce_cols4(void* __restrict__ partials, const void* __restrict__ src,
                                                      uint32_t groups, uint32_t out_count, Wheels<1> ow, Wheels<1> rw,
                                                      int op, uint32_t neutral, uint32_t total, uint32_t chunk_len) {
  using R = RedT<Tag>;
  using V4 = typename Vec4T<Tag>::type;
  __shared__ V4 part[4][64];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t g = blockIdx.x * 64 + lane;
  int64_t b[1];
  const bool dead = cell_base(ow, 4 * g, out_count, b);  // g >= groups reads as dead
  const Tag z = R::from_bits(neutral);
  V4 acc = {z, z, z, z};
  const uint32_t c0 = blockIdx.y * chunk_len, c1 = min(total, c0 + chunk_len);
  const uint32_t wlen = (chunk_len + 3) / 4;
  const uint32_t r_begin = min(c1, c0 + wave * wlen), r_end = min(c1, r_begin + wlen);
  if (!dead && r_begin < r_end) {
    // The op is dispatched once, outside the row loop, with 16 rows in flight (8192 x 8192 f32
    // columns: 4.64 -> 5.12 TB/s against a switch per element and 8 rows).
    switch (op) {
      case FO_RED_ADD:
        acc = cols4_rows<Tag, FO_RED_ADD>(src, rw, b[0], r_begin, r_end, acc);
        break;
      case FO_RED_MAX:
        acc = cols4_rows<Tag, FO_RED_MAX>(src, rw, b[0], r_begin, r_end, acc);
        break;
      case FO_RED_MIN:
        acc = cols4_rows<Tag, FO_RED_MIN>(src, rw, b[0], r_begin, r_end, acc);
        break;
      default:
        acc = cols4_rows<Tag, FO_RED_MUL>(src, rw, b[0], r_begin, r_end, acc);
        break;
    }
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && g < groups) {
    V4 t = part[0][lane];
#pragma unroll
    for (int w = 1; w < 4; ++w)
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] = R::apply(op, t[e], part[w][lane][e]);
    ((V4*)partials)[(int64_t)blockIdx.y * groups + g] = t;
  }
}

template <typename Tag>
__global__ void __launch_bounds__(kBlock) k_reduce_cols4_fold(void* dst, const void* __restrict__ partials,
                                                              uint32_t out_count, uint32_t nchunks, Wheels<1> ow, int op,
                                                              uint32_t identity) {
  using R = RedT<Tag>;
  const uint32_t o = blockIdx.x * kBlock + threadIdx.x;
  if (o >= out_count) return;
  int64_t b[1];
  const bool dead = cell_base(ow, o, out_count, b);
  auto acc = R::from_bits(identity);
  if (!dead) {
    uint32_t c = 0;
    for (; c + 8 <= nchunks; c += 8) {  // eight loads in flight, folded in chunk order
      decltype(R::load(partials, 0)) v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = R::load(partials, (int64_t)(c + u) * out_count + o);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = R::apply(op, acc, v[u]);
    }
    for (; c < nchunks; ++c) acc = R::apply(op, acc, R::load(partials, (int64_t)c * out_count + o));
  }
  R::store(dst, o, acc);
}

template <typename Tag>
void reduce_t(hipStream_t s, void* dst, const void* src, int64_t src_len, int64_t out_count, const Wheels<1>& ow,
              const Wheels<1>& rw, int op, uint32_t identity) {
  int64_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  require(total < (1ll << 31), "reduce: residue larger than 2^31");
  // Folds that must keep the emulator's exact serial order -- bf16 (`half` arithmetic rounds every
  // step, so any regrouping shows) and the saturating add (not associative) -- take the thread form
  // or, for a long residue contiguous in the source, the coalesced tile form. The other folds
  // (f32, and the integer ops, which are exact in any order) regroup a long residue for
  // parallelism: a wave per cell when the residue is contiguous, 64 cells x kSeg segments per block
  // when the cells are. For f32 that reassociates the sum, which BufStorage::reduce's own contract
  // accepts (buf.rs:316-330) and the f32 tolerance covers.
  constexpr bool is_f32 = std::is_same<Tag, float>::value || std::is_same<Tag, WidenedBf16>::value ||
                         std::is_same<Tag, RoundedBf16>::value;
  const bool exact_only = std::is_same<Tag, Bf16Red>::value || op == FO_RED_ADD_SAT;
  const bool res_contig = rw.n > 0 && rw.stride[0][0] == 1;
  const bool cells_contig = ow.n > 0 && ow.stride[0][0] == 1;
  // The op's neutral element (-0 for the f32 add, so that a -0 sum keeps its sign).
  uint32_t neutral = 0;
  switch (op) {
    case FO_RED_ADD:
      neutral = is_f32 ? 0x80000000u : 0u;
      break;
    case FO_RED_MAX:
      neutral = is_f32 ? 0xff800000u : 0x80000000u;
      break;
    case FO_RED_MIN:
      neutral = is_f32 ? 0x7f800000u : 0x7fffffffu;
      break;
    default:
      neutral = is_f32 ? 0x3f800000u : 1u;
      break;
  }
  if (!exact_only && total >= 64 && res_contig && out_count <= (1 << 20)) {
    hipLaunchKernelGGL(k_reduce_wave<Tag>, dim3(grid_for(out_count * 64)), dim3(kBlock), 0, s, dst, src, src_len,
                       (uint32_t)out_count, ow, rw, op, identity, neutral);
  } else if (!exact_only && total >= 64 && cells_contig) {
    hipLaunchKernelGGL(k_reduce_cols<Tag>, dim3((unsigned)((out_count + 63) / 64)), dim3(64 * kSeg), 0, s, dst, src,
                       src_len, (uint32_t)out_count, ow, rw, op, identity, neutral, (uint32_t)total);
  } else if (total >= 32 && res_contig && src_len > 0) {
    int64_t blocks = (out_count + 255) / 256;
    if (blocks > 65535ll * 16) blocks = 65535ll * 16;
    hipLaunchKernelGGL(k_reduce_tiled<Tag>, dim3((unsigned)blocks), dim3(256), 0, s, dst, src, src_len,
                       (uint32_t)out_count, ow, rw, op, identity, (uint32_t)total);
  } else if (rw.n == 1) {
    hipLaunchKernelGGL(k_reduce_strided<Tag>, dim3(grid_for(out_count)), dim3(kBlock), 0, s, dst, src, src_len,
                       (uint32_t)out_count, ow, (uint32_t)total, rw.stride[0][0], op, identity);
  } else {
    hipLaunchKernelGGL(k_reduce_thread<Tag>, dim3(grid_for(out_count)), dim3(kBlock), 0, s, dst, src, src_len,
                       (uint32_t)out_count, ow, rw, op, identity);
  }
  FO_HIP(hipGetLastError());
}

}  // namespace

namespace {
constexpr int64_t kColsTargetBlocks = 2048;

// The op's neutral element as bits (f32 or i32).
uint32_t red_neutral(bool f32, int op) {
  switch (op) {
    case FO_RED_ADD:
      return f32 ? 0x80000000u : 0u;
    case FO_RED_MAX:
      return f32 ? 0xff800000u : 0x80000000u;
    case FO_RED_MIN:
      return f32 ? 0x7f800000u : 0x7fffffffu;
    default:
      return f32 ? 0x3f800000u : 1u;
  }
}
}  // namespace

ReduceSplit plan_reduce_split(fo_dtype t, int op, const void* src, int64_t src_len, int64_t out_count,
                              const Wheels<1>& ow, const Wheels<1>& rw) {
  ReduceSplit p;
  if (!(t == FO_F32 || (t == FO_I32 && op != FO_RED_ADD_SAT))) return p;
  if (ow.n < 1 || rw.n < 1 || ow.stride[0][0] != 1 || ow.size[0] % 4 != 0 || ow.live[0] != ow.size[0]) return p;
  if (rw.stride[0][0] == 1 && out_count <= (1 << 20)) return p;  // a contiguous residue: the wave form
  if ((uintptr_t)src % 16 != 0) return p;
  int64_t total = 1, max_off = 0;
  for (int i = 0; i < ow.n; ++i) {
    if (i > 0 && ow.stride[0][i] % 4 != 0) return p;
    if (ow.live[i] > 0) max_off += (int64_t)(ow.live[i] - 1) * ow.stride[0][i];  // dead cells are never read
  }
  for (int i = 0; i < rw.n; ++i) {
    if (rw.stride[0][i] % 4 != 0 || rw.stride[0][i] < 0) return p;
    max_off += (int64_t)(rw.size[i] - 1) * rw.stride[0][i];
    total *= rw.size[i];
  }
  if (total < 64 || total >= (1ll << 31) || max_off >= src_len || out_count % 4 != 0) return p;
  const int64_t groups = out_count / 4, tiles = (groups + 63) / 64;
  int64_t nchunks = (kColsTargetBlocks + tiles - 1) / tiles;
  nchunks = std::max<int64_t>(1, std::min<int64_t>({nchunks, (total + 15) / 16, 65535}));  // >= 16 rows a chunk
  p.nchunks = nchunks;
  p.chunk_len = (total + nchunks - 1) / nchunks;
  p.nchunks = (total + p.chunk_len - 1) / p.chunk_len;
  p.scratch_bytes = (uint64_t)p.nchunks * out_count * 4;
  return p;
}

void launch_reduce_split(hipStream_t s, void* dst, const void* src, fo_dtype t, int64_t out_count, const Wheels<1>& ow,
                         const Wheels<1>& rw, int op, uint32_t identity, const ReduceSplit& p, void* scratch) {
  int64_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  const uint32_t groups = (uint32_t)(out_count / 4);
  const dim3 grid((groups + 63) / 64, (unsigned)p.nchunks);
  const unsigned fold_blocks = (unsigned)((out_count + kBlock - 1) / kBlock);
  const bool f32 = t == FO_F32;
  if (f32) {
    hipLaunchKernelGGL(k_reduce_cols4<float>, grid, dim3(256), 0, s, scratch, src, groups, (uint32_t)out_count, ow, rw,
                       op, red_neutral(true, op), (uint32_t)total, (uint32_t)p.chunk_len);
    hipLaunchKernelGGL(k_reduce_cols4_fold<float>, dim3(fold_blocks), dim3(kBlock), 0, s, dst, scratch,
                       (uint32_t)out_count, (uint32_t)p.nchunks, ow, op, identity);
  } else {
    hipLaunchKernelGGL(k_reduce_cols4<int32_t>, grid, dim3(256), 0, s, scratch, src, groups, (uint32_t)out_count, ow,
                       rw, op, red_neutral(false, op), (uint32_t)total, (uint32_t)p.chunk_len);
    hipLaunchKernelGGL(k_reduce_cols4_fold<int32_t>, dim3(fold_blocks), dim3(kBlock), 0, s, dst, scratch,
                       (uint32_t)out_count, (uint32_t)p.nchunks, ow, op, identity);
  }
  FO_HIP(hipGetLastError());
}

void launch_reduce(hipStream_t s, void* dst, const void* src, fo_dtype t, int64_t src_len, int64_t out_count,
                   const Wheels<1>& ow, const Wheels<1>& rw, int op, uint32_t identity) {
  switch (t) {
    case FO_F32:
      return reduce_t<float>(s, dst, src, src_len, out_count, ow, rw, op, identity);
    case FO_I32:
      return reduce_t<int32_t>(s, dst, src, src_len, out_count, ow, rw, op, identity);
    case FO_BF16:
      return reduce_t<Bf16Red>(s, dst, src, src_len, out_count, ow, rw, op, identity);
    default:
      throw InvalidArg("reduce: unsupported dtype");
  }
}

void launch_reduce_widened(hipStream_t s, void* dst, const void* src, bool via_bf16, int64_t src_len,
                           int64_t out_count, const Wheels<1>& ow, const Wheels<1>& rw, int op, uint32_t identity) {
  if (via_bf16)
    reduce_t<RoundedBf16>(s, dst, src, src_len, out_count, ow, rw, op, identity);
  else
    reduce_t<WidenedBf16>(s, dst, src, src_len, out_count, ow, rw, op, identity);
}

// ---------------------------------------------------------------------------------------------
// Generic contraction: one thread per output cell, products folded in residue wire order with
// separate multiply and add roundings -- the exact fold of contraction_in (buf.rs:428-445).
// ---------------------------------------------------------------------------------------------
namespace {

// The two 8-bit float operand types, distinct from each other and from uint8_t.
struct f8e4m3_t {
  uint8_t bits;
};
struct f8e5m2_t {
  uint8_t bits;
};

template <typename In, typename Acc>
struct MacT;
template <>
struct MacT<f8e4m3_t, float> {  // f8 operands, f32 accumulator (ContractionCast, cast.rs:357-363)
  static __device__ __forceinline__ float widen(f8e4m3_t v) { return f8e4m3_to_f32(v.bits); }
  static __device__ __forceinline__ float mac(float acc, float a, float b) { return __fadd_rn(acc, __fmul_rn(a, b)); }
};
template <>
struct MacT<f8e5m2_t, float> {
  static __device__ __forceinline__ float widen(f8e5m2_t v) { return f8e5m2_to_f32(v.bits); }
  static __device__ __forceinline__ float mac(float acc, float a, float b) { return __fadd_rn(acc, __fmul_rn(a, b)); }
};
template <>
struct MacT<uint16_t, float> {  // bf16 operands, f32 accumulator
  static __device__ __forceinline__ float widen(uint16_t v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ float mac(float acc, float a, float b) { return __fadd_rn(acc, __fmul_rn(a, b)); }
};
template <>
struct MacT<float, float> {
  static __device__ __forceinline__ float widen(float v) { return v; }
  static __device__ __forceinline__ float mac(float acc, float a, float b) { return __fadd_rn(acc, __fmul_rn(a, b)); }
};
template <>
struct MacT<int8_t, int32_t> {
  static __device__ __forceinline__ int32_t widen(int8_t v) { return (int32_t)v; }
  static __device__ __forceinline__ int32_t mac(int32_t acc, int32_t a, int32_t b) {
    return (int32_t)((uint32_t)acc + (uint32_t)a * (uint32_t)b);
  }
};
template <>
struct MacT<int32_t, int32_t> {
  static __device__ __forceinline__ int32_t widen(int32_t v) { return v; }
  static __device__ __forceinline__ int32_t mac(int32_t acc, int32_t a, int32_t b) {
    return (int32_t)((uint32_t)acc + (uint32_t)a * (uint32_t)b);
  }
};

template <typename In, typename Acc, typename Out>
__device__ __forceinline__ Out narrow(Acc a);
template <>
__device__ __forceinline__ uint16_t narrow<uint16_t, float, uint16_t>(float a) {
  return f32_to_bf16(a);
}
template <>
__device__ __forceinline__ float narrow<uint16_t, float, float>(float a) {
  return a;
}
template <>
__device__ __forceinline__ float narrow<float, float, float>(float a) {
  return a;
}
template <>
__device__ __forceinline__ f8e4m3_t narrow<f8e4m3_t, float, f8e4m3_t>(float a) {
  return f8e4m3_t{f32_to_f8e4m3(a)};
}
template <>
__device__ __forceinline__ float narrow<f8e4m3_t, float, float>(float a) {
  return a;
}
template <>
__device__ __forceinline__ f8e5m2_t narrow<f8e5m2_t, float, f8e5m2_t>(float a) {
  return f8e5m2_t{f32_to_f8e5m2(a)};
}
template <>
__device__ __forceinline__ float narrow<f8e5m2_t, float, float>(float a) {
  return a;
}
template <>
__device__ __forceinline__ int8_t narrow<int8_t, int32_t, int8_t>(int32_t a) {
  return (int8_t)a;
}
template <>
__device__ __forceinline__ int32_t narrow<int8_t, int32_t, int32_t>(int32_t a) {
  return a;
}
template <>
__device__ __forceinline__ int32_t narrow<int32_t, int32_t, int32_t>(int32_t a) {
  return a;
}

template <typename In, typename Acc, typename Out>
__global__ void __launch_bounds__(kBlock) k_contract_generic(Out* __restrict__ out, const In* __restrict__ lhs,
                                                             const In* __restrict__ rhs, int64_t lhs_len,
                                                             int64_t rhs_len, uint32_t out_count, Wheels<2> ow,
                                                             Wheels<2> rw) {
  using M = MacT<In, Acc>;
  uint32_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  for (uint32_t o = blockIdx.x * kBlock + threadIdx.x; o < out_count; o += gridDim.x * kBlock) {
    int64_t bl = 0, br = 0;
    uint32_t q = o;
    bool dead = false;
    for (int i = 0; i < ow.n; ++i) {
      uint32_t nq = ow.div[i].div(q);
      uint32_t d = q - nq * ow.size[i];
      dead |= d >= ow.live[i];
      bl += (int64_t)d * ow.stride[0][i];
      br += (int64_t)d * ow.stride[1][i];
      q = nq;
    }
    Acc acc = Acc(0);
    if (dead) {  // a padding cell has no reads and keeps its zero (buf.rs:425-437)
      out[o] = narrow<In, Acc, Out>(acc);
      continue;
    }
    uint32_t digit[kMaxWheels] = {};
    int64_t off[2] = {bl, br};
    // kBatch pairs of reads are issued before they are folded, in wire order.
    for (uint32_t r0 = 0; r0 < total; r0 += kBatch) {
      In va[kBatch], vb[kBatch];
      bool ok[kBatch];
      int64_t al[kBatch], ar[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const bool in = r0 + u < total;
        ok[u] = in && off[0] < lhs_len && off[1] < rhs_len;
        al[u] = ok[u] ? off[0] : 0;
        ar[u] = ok[u] ? off[1] : 0;
        if (in) odometer_step(rw, digit, off);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {  // all reads in flight together
        va[u] = lhs[al[u]];
        vb[u] = rhs[ar[u]];
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (ok[u]) acc = M::mac(acc, M::widen(va[u]), M::widen(vb[u]));
    }
    out[o] = narrow<In, Acc, Out>(acc);
  }
}

// Batched dot products: every output wheel reads both operands (or neither: padding) and the
// residue is one run of K contiguous elements in both, so each output cell folds two rows. One lane
// per cell folds its K products in k order -- k_contract_generic's arithmetic and order -- reading
// 16 bytes of each row at a time, four such pairs in flight ahead of the fold (vec: every row start
// 16-byte aligned). The MNIST fc1 stream (mnist/mod.rs:8-34) issues this shape: 256 cells of one
// 800-long dot product, the rhs a copy of the input per cell.
template <typename In, typename Acc, typename Out>
__global__ void __launch_bounds__(kBlock) k_contract_dot(Out* __restrict__ out, const In* __restrict__ lhs,
                                                         const In* __restrict__ rhs, uint32_t out_count,
                                                         Wheels<2> ow, uint32_t K, int32_t vec) {
  using M = MacT<In, Acc>;
  constexpr int V = 16 / (int)sizeof(In);  // elements per 16-byte read
  constexpr int U = 4;                      // 16-byte pairs per batch
  const uint32_t o = blockIdx.x * kBlock + threadIdx.x;
  if (o >= out_count) return;
  int64_t bl = 0, br = 0;
  uint32_t q = o;
  bool dead = false;
  for (int i = 0; i < ow.n; ++i) {
    const uint32_t nq = ow.div[i].div(q);
    const uint32_t d = q - nq * ow.size[i];
    dead |= d >= ow.live[i];
    bl += (int64_t)d * ow.stride[0][i];
    br += (int64_t)d * ow.stride[1][i];
    q = nq;
  }
  Acc acc = Acc(0);
  if (!dead) {  // a padding cell has no reads and keeps its zero (buf.rs:425-437)
    const In* a = lhs + bl;
    const In* b = rhs + br;
    uint32_t k = 0;
    if (vec) {
      typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
      i32x4_t va[U], vb[U];
      auto load = [&](uint32_t k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          va[u] = *(const i32x4_t*)(a + k0 + u * V);
          vb[u] = *(const i32x4_t*)(b + k0 + u * V);
        }
      };
      if (K >= (uint32_t)(U * V)) load(0);
      for (; k + U * V <= K; k += U * V) {
        i32x4_t ca[U], cb[U];
#pragma unroll
        for (int u = 0; u < U; ++u) ca[u] = va[u], cb[u] = vb[u];
        if (k + 2 * U * V <= K) load(k + U * V);  // the next batch in flight during this fold
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const In* ea = (const In*)&ca[u];
          const In* eb = (const In*)&cb[u];
#pragma unroll
          for (int e = 0; e < V; ++e) acc = M::mac(acc, M::widen(ea[e]), M::widen(eb[e]));
        }
      }
    }
    for (; k < K; ++k) acc = M::mac(acc, M::widen(a[k]), M::widen(b[k]));
  }
  out[o] = narrow<In, Acc, Out>(acc);
}

// The product and the sum of contraction_in, as separate roundings (no fused multiply-add).
__device__ __forceinline__ float mul_of(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_of(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ int32_t mul_of(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
__device__ __forceinline__ int32_t add_of(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }

// The same dot products with the reads spread over a block: 256 threads stage the products of 16
// cells (one multiply each, MacT's rounding) in LDS, 512 positions of each row at a time and the next
// 512 loading while the current ones are folded; lane c of wave 0 then adds cell c's products in k
// order. The multiplies do not depend on the running sum, so only the adds stay serial, and the
// result is the lane-per-cell kernel's bit for bit. Every row start is 16-byte aligned (vec).
constexpr int kDotCells = 16;   // cells per block
constexpr int kDotChunk = 512;  // positions per stage
template <typename In, typename Acc, typename Out>
__global__ void __launch_bounds__(kBlock) k_contract_dot_staged(Out* __restrict__ out, const In* __restrict__ lhs,
                                                                const In* __restrict__ rhs, uint32_t out_count,
                                                                Wheels<2> ow, uint32_t K) {
  static_assert(kBlock == kDotCells * 16, "16 threads stage each cell");
  using M = MacT<In, Acc>;
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4_t;
  constexpr int V = 16 / (int)sizeof(In);       // elements per 16-byte read
  constexpr int NJ = kDotChunk / (16 * V);      // 16-byte reads per operand per thread per stage
  constexpr int ROW = kDotChunk + 4;            // padded row: lane c's reads start on distinct banks
  __shared__ Acc prod[2][kDotCells][ROW];
  const int t = threadIdx.x, sub = t & 15, cl = t >> 4;
  const uint32_t cell = blockIdx.x * kDotCells + cl;
  int64_t bl = 0, br = 0;
  bool dead = cell >= out_count;
  if (!dead) {
    uint32_t q = cell;
    for (int i = 0; i < ow.n; ++i) {
      const uint32_t nq = ow.div[i].div(q);
      const uint32_t d = q - nq * ow.size[i];
      dead |= d >= ow.live[i];
      bl += (int64_t)d * ow.stride[0][i];
      br += (int64_t)d * ow.stride[1][i];
      q = nq;
    }
  }
  const In* a = lhs + bl;
  const In* b = rhs + br;
  i32x4_t va[NJ], vb[NJ];
  auto load = [&](uint32_t k0) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t e = k0 + (uint32_t)(j * 16 + sub) * V;
      if (!dead && e + V <= K) {
        va[j] = *(const i32x4_t*)(a + e);
        vb[j] = *(const i32x4_t*)(b + e);
      } else if (!dead && e < K) {  // the ragged end of a row, element by element
        In ta[V], tb[V];
#pragma unroll
        for (int v = 0; v < V; ++v) ta[v] = e + v < K ? a[e + v] : In(0), tb[v] = e + v < K ? b[e + v] : In(0);
        va[j] = *(const i32x4_t*)ta;
        vb[j] = *(const i32x4_t*)tb;
      }
    }
  };
  const uint32_t stages = (K + kDotChunk - 1) / kDotChunk;
  const bool folds = t < kDotCells && blockIdx.x * kDotCells + t < out_count;
  bool fold_dead = false;
  if (folds) {  // lane t folds cell blockIdx.x * 16 + t; its liveness, decoded again
    uint32_t q = blockIdx.x * kDotCells + t;
    for (int i = 0; i < ow.n; ++i) {
      const uint32_t nq = ow.div[i].div(q);
      fold_dead |= q - nq * ow.size[i] >= ow.live[i];
      q = nq;
    }
  }
  Acc acc = Acc(0);
  load(0);
  for (uint32_t s = 0; s < stages; ++s) {
    const uint32_t k0 = s * kDotChunk;
    Acc* row = prod[s & 1][cl];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const uint32_t e = (uint32_t)(j * 16 + sub) * V;
      if (!dead && k0 + e < K) {
        const In* ea = (const In*)&va[j];
        const In* eb = (const In*)&vb[j];
#pragma unroll
        for (int v = 0; v < V; v += 4) {
          Acc p4[4];
#pragma unroll
          for (int w = 0; w < 4; ++w) p4[w] = mul_of(M::widen(ea[v + w]), M::widen(eb[v + w]));
          *(i32x4_t*)(row + e + v) = *(const i32x4_t*)p4;
        }
      }
    }
    __syncthreads();
    if (s + 1 < stages) load(k0 + kDotChunk);  // in flight while this stage is folded
    if (folds && !fold_dead) {
      const Acc* pr = prod[s & 1][t];
      const uint32_t klen = min((uint32_t)kDotChunk, K - k0);
      uint32_t k = 0;
      for (; k + 32 <= klen; k += 32) {  // eight reads in flight ahead of the adds
        i32x4_t p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = *(const i32x4_t*)(pr + k + 4 * u);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const Acc* pe = (const Acc*)&p[u];
          acc = add_of(add_of(add_of(add_of(acc, pe[0]), pe[1]), pe[2]), pe[3]);
        }
      }
      for (; k + 4 <= klen; k += 4) {
        const i32x4_t p = *(const i32x4_t*)(pr + k);
        const Acc* pe = (const Acc*)&p;
        acc = add_of(add_of(add_of(add_of(acc, pe[0]), pe[1]), pe[2]), pe[3]);
      }
      for (; k < klen; ++k) acc = add_of(acc, pr[k]);
    }
  }
  if (folds) out[blockIdx.x * kDotCells + t] = narrow<In, Acc, Out>(acc);  // a padding cell keeps zero
}


// Affine contractions on the vector units (f32, i32, and bf16 or i8 operands widened as they are
// staged): one wave per T x T cells of a
// batch cell (T = 8 R), lane (ty, tx) = (lane / 8, lane % 8) holding rows R ty .. R ty + R - 1 and
// columns R tx .. R tx + R - 1 (R = 4, or 2 when 32 x 32 tiles would leave most of the chip idle).
// K goes through LDS 32 positions at a time, k-major (a lane's rows or columns are one 8- or 16-byte
// read), the next 32 loading into registers while the current ones are folded. A stage's loads run
// k-fastest across lanes for an operand whose k stride is 1, else row-fastest. Each cell adds
// mul(a, b) to its sum in k order from zero: contraction_in's arithmetic, bit for bit.
constexpr int kSimtK = 32;  // contracted positions per stage
template <typename In, typename Acc, typename Out, int R>
__global__ void __launch_bounds__(64) k_contract_simt(Out* __restrict__ out, const In* __restrict__ lhs,
                                                      const In* __restrict__ rhs, GemmDesc d, int64_t sa, int64_t sb) {
  using M = MacT<In, Acc>;
  constexpr int T = 8 * R;       // rows and columns per wave
  constexpr int NE = T / 2;      // elements of each operand per lane per stage
  typedef Acc accr_t __attribute__((ext_vector_type(R)));
  __shared__ Acc As[kSimtK][T + 4];
  __shared__ Acc Bs[kSimtK][T + 4];
  const int lane = threadIdx.x, ty = lane >> 3, tx = lane & 7;
  const int64_t m0 = (int64_t)blockIdx.y * T, n0 = (int64_t)blockIdx.x * T, bb = blockIdx.z;
  // Lane element i of a stage is tile position (r0 + i dr, kk + i dk): k fixed and rows every two
  // (k-fast), or the row fixed and k every 64 / T (row-fast).
  struct Walk {
    const In* p;    // the lane's first element
    int64_t step;   // elements between its consecutive ones
    int64_t kstep;  // elements per contracted position
    int r0, kk, dr, dk;
  };
  auto walk = [&](const In* base, int64_t row0, int64_t ld, int64_t sk) {
    Walk w;
    if (sk == 1) w.kk = lane & 31, w.r0 = lane >> 5, w.dr = 2, w.dk = 0;
    else w.r0 = lane % T, w.kk = lane / T, w.dr = 0, w.dk = 64 / T;
    w.p = base + (row0 + w.r0) * ld + w.kk * sk;
    w.step = w.dr * ld + w.dk * sk;
    w.kstep = sk;
    return w;
  };
  const Walk wa = walk(lhs + bb * d.a_batch, m0, d.lda, sa), wb = walk(rhs + bb * d.b_batch, n0, d.ldb, sb);
  const int64_t ra_rows = d.M - m0, rb_rows = d.N - n0;
  In ra[NE], rb[NE];
  auto load = [&](int64_t k0) {
    const int64_t kl = d.K - k0;
    const In* pa = wa.p + k0 * wa.kstep;
    const In* pb = wb.p + k0 * wb.kstep;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      ra[i] = (wa.r0 + i * wa.dr < ra_rows && wa.kk + i * wa.dk < kl) ? pa[i * wa.step] : In(0);
      rb[i] = (wb.r0 + i * wb.dr < rb_rows && wb.kk + i * wb.dk < kl) ? pb[i * wb.step] : In(0);
    }
  };
  Acc acc[R][R];
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < R; ++j) acc[i][j] = Acc(0);
  auto step = [&](int k) {
    const accr_t a = *(const accr_t*)&As[k][ty * R];
    const accr_t b = *(const accr_t*)&Bs[k][tx * R];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int j = 0; j < R; ++j) acc[i][j] = add_of(acc[i][j], mul_of(a[i], b[j]));
  };
  load(0);
  for (int64_t k0 = 0; k0 < d.K; k0 += kSimtK) {
    __syncthreads();  // the previous stage's reads are done
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      As[wa.kk + i * wa.dk][wa.r0 + i * wa.dr] = M::widen(ra[i]);
      Bs[wb.kk + i * wb.dk][wb.r0 + i * wb.dr] = M::widen(rb[i]);
    }
    __syncthreads();
    if (k0 + kSimtK < d.K) load(k0 + kSimtK);
    if (d.K - k0 >= kSimtK) {
#pragma unroll
      for (int k = 0; k < kSimtK; ++k) step(k);  // unrolled: the LDS reads run ahead of the adds
    } else {
      for (int k = 0; k < (int)(d.K - k0); ++k) step(k);
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int j = 0; j < R; ++j) {
      const int64_t m = m0 + ty * R + i, n = n0 + tx * R + j;
      if (m < d.M && n < d.N) out[bb * d.c_batch + m * d.ldc_m + n * d.ldc_n] = narrow<In, Acc, Out>(acc[i][j]);
    }
}

// The same fold with coalesced reads: one wave per 64 consecutive output cells, the residue taken
// 64 positions at a time. Lane l decodes residue position r0 + l; for each of the wave's cells in
// turn every lane reads that cell's operands at position r0 + l (consecutive lanes, consecutive
// positions when the residue is contiguous) and leaves the product in LDS; then lane c folds its
// cell's 64 products in residue order. The arithmetic and its order are k_contract_generic's.
constexpr int kTileW = 4;  // waves per block
template <typename In, typename Acc, typename Out>
__global__ void __launch_bounds__(64 * kTileW) k_contract_tiled(Out* __restrict__ out, const In* __restrict__ lhs,
                                                              const In* __restrict__ rhs, int64_t lhs_len,
                                                              int64_t rhs_len, uint32_t out_count, Wheels<2> ow,
                                                              Wheels<2> rw, uint32_t total) {
  using M = MacT<In, Acc>;
  __shared__ Acc prod[kTileW][64][65];     // a padded row per cell: lane c's reads hit distinct banks
  __shared__ uint64_t valid[kTileW][64];   // per cell, the residue positions whose reads are in range
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (uint64_t g0 = ((uint64_t)blockIdx.x * kTileW + wave) * 64; g0 < out_count;
       g0 += (uint64_t)gridDim.x * kTileW * 64) {
    const uint32_t o = (uint32_t)g0 + lane;
    int64_t b[2];
    const bool dead = cell_base(ow, o, out_count, b);
    Acc acc = Acc(0);
    for (uint32_t r0 = 0; r0 < total; r0 += 64) {
      const bool rin = r0 + lane < total;
      int64_t d[2] = {0, 0};
      if (rin) {
        uint32_t q = r0 + lane;
        for (int i = 0; i < rw.n; ++i) {
          const uint32_t nq = rw.div[i].div(q);
          const uint32_t dg = q - nq * rw.size[i];
          d[0] += (int64_t)dg * rw.stride[0][i];
          d[1] += (int64_t)dg * rw.stride[1][i];
          q = nq;
        }
      }
      // 16 cells at a time: their reads are all issued before the first is used.
#pragma unroll
      for (int cg = 0; cg < 64; cg += 16) {
        In va[16], vb[16];
        bool ok[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int64_t al = readlane64(b[0], cg + u) + d[0], ar = readlane64(b[1], cg + u) + d[1];
          ok[u] = rin && al < lhs_len && ar < rhs_len;
          va[u] = lhs[ok[u] ? al : 0];
          vb[u] = rhs[ok[u] ? ar : 0];
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          prod[wave][cg + u][lane] = mul_of(M::widen(va[u]), M::widen(vb[u]));
          const uint64_t mask = __ballot(ok[u]);
          if (lane == 0) valid[wave][cg + u] = mask;
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint64_t vm = valid[wave][lane];
      const int cnt = (int)min(64u, total - r0);
      if (!dead)
        for (int j = 0; j < cnt; ++j)
          if ((vm >> j) & 1u) acc = add_of(acc, prod[wave][lane][j]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    if (o < out_count) out[o] = narrow<In, Acc, Out>(acc);
  }
}

template <typename In, typename Acc, typename Out>
void contract_t(hipStream_t s, void* out, const void* lhs, const void* rhs, int64_t ll, int64_t rl, int64_t n,
                const Wheels<2>& ow, const Wheels<2>& rw) {
  int64_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  if (total >= 32 && ll > 0 && rl > 0 && rw.n > 0 && (rw.stride[0][0] == 1 || rw.stride[1][0] == 1)) {
    // Long residues contiguous in an operand: the tile form (consecutive lanes read consecutive
    // residue positions, and a chunk's reads are in flight together). A strided residue keeps the
    // thread form, where consecutive lanes are consecutive output cells.
    int64_t blocks = (n + kTileW * 64 - 1) / (kTileW * 64);
    if (blocks > 65535ll * 16) blocks = 65535ll * 16;
    hipLaunchKernelGGL((k_contract_tiled<In, Acc, Out>), dim3((unsigned)blocks), dim3(64 * kTileW), 0, s, (Out*)out,
                       (const In*)lhs, (const In*)rhs, ll, rl, (uint32_t)n, ow, rw, (uint32_t)total);
  } else {
    hipLaunchKernelGGL((k_contract_generic<In, Acc, Out>), dim3(grid_for(n)), dim3(kBlock), 0, s, (Out*)out,
                       (const In*)lhs, (const In*)rhs, ll, rl, (uint32_t)n, ow, rw);
  }
  FO_HIP(hipGetLastError());
}

template <typename In, typename Acc, typename Out>
void contract_dot_t(hipStream_t s, void* out, const void* lhs, const void* rhs, int64_t n, const Wheels<2>& ow,
                    int64_t K, bool vec) {
  if (vec && K >= 64)
    hipLaunchKernelGGL((k_contract_dot_staged<In, Acc, Out>), dim3((unsigned)((n + kDotCells - 1) / kDotCells)),
                       dim3(kBlock), 0, s, (Out*)out, (const In*)lhs, (const In*)rhs, (uint32_t)n, ow, (uint32_t)K);
  else
    hipLaunchKernelGGL((k_contract_dot<In, Acc, Out>), dim3((unsigned)((n + kBlock - 1) / kBlock)), dim3(kBlock), 0, s,
                       (Out*)out, (const In*)lhs, (const In*)rhs, (uint32_t)n, ow, (uint32_t)K, (int32_t)vec);
  FO_HIP(hipGetLastError());
}

}  // namespace

template <typename In, typename Acc, typename Out>
void simt_t(hipStream_t s, void* out, const void* lhs, const void* rhs, const GemmDesc& d, int64_t sa, int64_t sb, int T) {
  const dim3 grid((unsigned)((d.N + T - 1) / T), (unsigned)((d.M + T - 1) / T), (unsigned)d.batch);
  if (T == 32)
    hipLaunchKernelGGL((k_contract_simt<In, Acc, Out, 4>), grid, dim3(64), 0, s, (Out*)out, (const In*)lhs,
                       (const In*)rhs, d, sa, sb);
  else
    hipLaunchKernelGGL((k_contract_simt<In, Acc, Out, 2>), grid, dim3(64), 0, s, (Out*)out, (const In*)lhs,
                       (const In*)rhs, d, sa, sb);
}

bool launch_contraction_simt(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t, fo_dtype out_t,
                             const GemmDesc& d, int64_t sa, int64_t sb) {
  if (d.M <= 0 || d.N <= 0 || d.K <= 0 || d.batch <= 0 || d.batch > 65535) return false;
  // 32 x 32 cells a wave when that gives at least two waves per CU, else 16 x 16.
  const int64_t waves32 = ((d.M + 31) / 32) * ((d.N + 31) / 32) * d.batch;
  const int T = waves32 >= 512 ? 32 : 16;
  if ((d.M + T - 1) / T > 65535 || (d.N + T - 1) / T > (1ll << 31) - 1) return false;
  if (in_t == FO_F32 && out_t == FO_F32) simt_t<float, float, float>(s, out, lhs, rhs, d, sa, sb, T);
  else if (in_t == FO_I32 && out_t == FO_I32) simt_t<int32_t, int32_t, int32_t>(s, out, lhs, rhs, d, sa, sb, T);
  else if (in_t == FO_BF16 && out_t == FO_F32) simt_t<uint16_t, float, float>(s, out, lhs, rhs, d, sa, sb, T);
  else if (in_t == FO_BF16 && out_t == FO_BF16) simt_t<uint16_t, float, uint16_t>(s, out, lhs, rhs, d, sa, sb, T);
  else if (in_t == FO_I8 && out_t == FO_I32) simt_t<int8_t, int32_t, int32_t>(s, out, lhs, rhs, d, sa, sb, T);
  else if (in_t == FO_I8 && out_t == FO_I8) simt_t<int8_t, int32_t, int8_t>(s, out, lhs, rhs, d, sa, sb, T);
  else
    return false;
  FO_HIP(hipGetLastError());
  return true;
}

bool launch_contraction_dot(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t, fo_dtype out_t,
                            int64_t n, const Wheels<2>& ow, int64_t K, bool vec) {
  if (n <= 0 || n >= (1ll << 31) || K >= (1ll << 31)) return false;
  if (in_t == FO_BF16 && out_t == FO_BF16) return contract_dot_t<uint16_t, float, uint16_t>(s, out, lhs, rhs, n, ow, K, vec), true;
  if (in_t == FO_BF16 && out_t == FO_F32) return contract_dot_t<uint16_t, float, float>(s, out, lhs, rhs, n, ow, K, vec), true;
  if (in_t == FO_F32 && out_t == FO_F32) return contract_dot_t<float, float, float>(s, out, lhs, rhs, n, ow, K, vec), true;
  if (in_t == FO_I8 && out_t == FO_I8) return contract_dot_t<int8_t, int32_t, int8_t>(s, out, lhs, rhs, n, ow, K, vec), true;
  if (in_t == FO_I8 && out_t == FO_I32) return contract_dot_t<int8_t, int32_t, int32_t>(s, out, lhs, rhs, n, ow, K, vec), true;
  if (in_t == FO_I32 && out_t == FO_I32) return contract_dot_t<int32_t, int32_t, int32_t>(s, out, lhs, rhs, n, ow, K, vec), true;
  return false;
}

void launch_contraction_generic(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t,
                                fo_dtype out_t, int64_t ll, int64_t rl, int64_t n, const Wheels<2>& ow,
                                const Wheels<2>& rw) {
  int64_t total = 1;
  for (int i = 0; i < rw.n; ++i) total *= rw.size[i];
  require(total < (1ll << 31), "contraction: contracted extent larger than 2^31");
  if (in_t == FO_BF16 && out_t == FO_BF16) return contract_t<uint16_t, float, uint16_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_BF16 && out_t == FO_F32) return contract_t<uint16_t, float, float>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_F32) return contract_t<float, float, float>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_F8E4M3 && out_t == FO_F8E4M3)
    return contract_t<f8e4m3_t, float, f8e4m3_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_F8E4M3 && out_t == FO_F32) return contract_t<f8e4m3_t, float, float>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_F8E5M2 && out_t == FO_F8E5M2)
    return contract_t<f8e5m2_t, float, f8e5m2_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_F8E5M2 && out_t == FO_F32) return contract_t<f8e5m2_t, float, float>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_I8 && out_t == FO_I8) return contract_t<int8_t, int32_t, int8_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_I8 && out_t == FO_I32) return contract_t<int8_t, int32_t, int32_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  if (in_t == FO_I32) return contract_t<int32_t, int32_t, int32_t>(s, out, lhs, rhs, ll, rl, n, ow, rw);
  throw InvalidArg("contraction: unsupported dtype pair");
}

}  // namespace fo

namespace fo {

void launch_gather(hipStream_t s, void* dst, const void* src, const int32_t* idx, int64_t elem_bytes,
                   int64_t payload, int64_t slots, int64_t axis_size, int32_t div, const Wheels<1>& ws,
                   const Wheels<1>& wd, int ws_slot_wheels, int wd_slot_wheels, int32_t* flag) {
  const int V = (int)(16 / elem_bytes);
  if (((uintptr_t)dst | (uintptr_t)src) % 16 == 0 && payload_vec_ok(ws, ws_slot_wheels, V) &&
      payload_vec_ok(wd, wd_slot_wheels, V)) {
    const uint32_t nch = (uint32_t)(payload / V), total = (uint32_t)(nch * slots);
    dim3 g(grid_for(total)), b(kBlock);
    const FastDiv cdiv(nch);
    if (V == 8)
      hipLaunchKernelGGL(k_gather_vec<8>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, total, cdiv,
                         (uint32_t)slots, (uint32_t)axis_size, div, ws, wd, flag);
    else if (V == 4)
      hipLaunchKernelGGL(k_gather_vec<4>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, total, cdiv,
                         (uint32_t)slots, (uint32_t)axis_size, div, ws, wd, flag);
    else
      hipLaunchKernelGGL(k_gather_vec<16>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, total,
                         cdiv, (uint32_t)slots, (uint32_t)axis_size, div, ws, wd, flag);
    FO_HIP(hipGetLastError());
    return;
  }
  const uint32_t total = (uint32_t)(payload * slots);
  dim3 g(grid_for(total)), b(kBlock);
  const FastDiv rdiv((uint32_t)slots);
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(k_gather<uint8_t>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, idx, total, rdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    case 2:
      hipLaunchKernelGGL(k_gather<uint16_t>, g, b, 0, s, (uint16_t*)dst, (const uint16_t*)src, idx, total, rdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    case 4:
      hipLaunchKernelGGL(k_gather<uint32_t>, g, b, 0, s, (uint32_t*)dst, (const uint32_t*)src, idx, total, rdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    default:
      throw InvalidArg("gather: unsupported element size");
  }
  FO_HIP(hipGetLastError());
}

void launch_scatter(hipStream_t s, void* dst, const void* src, const int32_t* idx, int64_t elem_bytes,
                    int64_t payload, int64_t keys, int64_t axis_size, int32_t div, const Wheels<1>& ws,
                    const Wheels<1>& wd, int ws_slot_wheels, int wd_slot_wheels, uint64_t* win, uint32_t gen,
                    int32_t* flag) {
  const uint64_t tag = (uint64_t)gen << 32;
  if (win) {  // without winner words (one key slot: no target is written twice) the copy checks the indices
    hipLaunchKernelGGL(k_scatter_winners, dim3(grid_for(keys)), dim3(kBlock), 0, s, idx, (uint32_t)keys,
                       (uint32_t)axis_size, div, win, tag, flag);
    FO_HIP(hipGetLastError());
  }
  const int V = (int)(16 / elem_bytes);
  if (((uintptr_t)dst | (uintptr_t)src) % 16 == 0 && payload_vec_ok(ws, ws_slot_wheels, V) &&
      payload_vec_ok(wd, wd_slot_wheels, V)) {
    const uint32_t nch = (uint32_t)(payload / V), total = (uint32_t)(nch * keys);
    dim3 g(grid_for(((int64_t)total + kChunkRuns - 1) / kChunkRuns)), b(kBlock);
    const FastDiv cdiv(nch);
    if (V == 8)
      hipLaunchKernelGGL(k_scatter_vec<8>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, win, tag,
                         total, cdiv, (uint32_t)keys, (uint32_t)axis_size, div, ws, wd, flag);
    else if (V == 4)
      hipLaunchKernelGGL(k_scatter_vec<4>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, win, tag,
                         total, cdiv, (uint32_t)keys, (uint32_t)axis_size, div, ws, wd, flag);
    else
      hipLaunchKernelGGL(k_scatter_vec<16>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, elem_bytes, idx, win,
                         tag, total, cdiv, (uint32_t)keys, (uint32_t)axis_size, div, ws, wd, flag);
    FO_HIP(hipGetLastError());
    return;
  }
  const uint32_t total = (uint32_t)(payload * keys);
  dim3 g(grid_for(total)), b(kBlock);
  const FastDiv kdiv((uint32_t)keys);
  switch (elem_bytes) {
    case 1:
      hipLaunchKernelGGL(k_scatter<uint8_t>, g, b, 0, s, (uint8_t*)dst, (const uint8_t*)src, idx, win, tag, total, kdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    case 2:
      hipLaunchKernelGGL(k_scatter<uint16_t>, g, b, 0, s, (uint16_t*)dst, (const uint16_t*)src, idx, win, tag, total, kdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    case 4:
      hipLaunchKernelGGL(k_scatter<uint32_t>, g, b, 0, s, (uint32_t*)dst, (const uint32_t*)src, idx, win, tag, total, kdiv,
                         (uint32_t)axis_size, div, ws, wd, flag);
      break;
    default:
      throw InvalidArg("scatter: unsupported element size");
  }
  FO_HIP(hipGetLastError());
}

}  // namespace fo
