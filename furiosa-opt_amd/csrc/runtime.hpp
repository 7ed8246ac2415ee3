// Internal runtime types behind the C ABI handles, and the kernel launchers each kernel file
// exports to the ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <vector>

#include "../../include/furiosa_hip.h"
#include "common.hpp"
#include "mapping.hpp"

// Device memory cache of one runtime. Blocks freed by fo_buffer_free return here and are handed out
// again only to buffers of the same runtime, whose every op is ordered on the runtime's one stream:
// work enqueued with the old owner completes before any work of the new one starts, so neither
// the free nor the reuse waits for the device. A pool outlives its runtime while buffers of it
// remain; those then release their blocks directly.
struct fo_graph_mem;
struct fo_buffer;
struct fo_pool {
  std::mutex mu;
  int device = 0;
  bool orphaned = false;                  // the runtime is gone: free blocks directly
  std::multimap<uint64_t, void*> cached;  // free blocks by capacity
  uint64_t cached_bytes = 0;
  static constexpr uint64_t kMaxCached = 8ull << 30;
  std::unordered_set<fo_buffer*> unfilled;  // live buffers whose deferred zero fill has not run
  std::shared_ptr<fo_graph_mem> recording;  // set while the runtime records a graph
  // Returns a block to the cache, or frees it (after the device drains) when the cache is full or
  // the runtime is gone.
  void release(void* ptr, uint64_t capacity);
};

// The device blocks a recorded graph's kernels touch: every block handed out while recording
// (outputs, intermediates, scratch, scatter winner words) and the blocks of buffers freed while
// recording. They stay out of the pool's cache while the graph or any buffer born in the recording
// lives, so a launch never writes memory that another buffer holds; the last holder returns them.
struct fo_graph_mem {
  std::shared_ptr<fo_pool> pool;
  std::vector<std::pair<uint64_t, void*>> blocks;       // (capacity, address), each once
  std::multimap<uint64_t, void*> reuse;                 // freed while recording: later allocations take them
  std::vector<std::shared_ptr<fo_graph_mem>> keep;      // earlier recordings' blocks freed in this one
  void* scratch = nullptr;                              // the recording's op scratch (grown by new blocks)
  uint64_t scratch_bytes = 0;
  ~fo_graph_mem() {
    for (auto& b : blocks) pool->release(b.second, b.first);
  }
};

struct fo_runtime {
  int device = 0;
  std::shared_ptr<fo_pool> pool;
  hipStream_t stream = nullptr;
  hipEvent_t events[16] = {};
  int cus = 0;
  std::string arch;
  void* scratch = nullptr;  // device scratch for ops that need working memory (grown on demand)
  uint64_t scratch_bytes = 0;
  int32_t* err_host = nullptr;  // pinned, device-mapped error word: kernels set it only on failure
  int32_t* err_dev = nullptr;   // its device address
  // Scatter's last-key-per-target words (see k_scatter_winners): zeroed when allocated, then tagged
  // with a per-call generation instead of cleared per call.
  uint64_t* scatter_win = nullptr;
  uint64_t scatter_win_slots = 0;
  uint32_t scatter_gen = 0;
  uint32_t err_ops = 0;  // ops that may have set it since the last check: bit 0 gather, 1 scatter, 2 zip3_slots
  // Trace spans (fo_runtime_set_trace): while a sink is set, every op brackets its launches with a
  // pair of events; the spans are read back and handed to the sink at the next synchronize.
  fo_trace_sink trace_sink = nullptr;
  fo_trace_done trace_done = nullptr;
  void* trace_ctx = nullptr;
  hipEvent_t trace_base = nullptr;
  struct Span {
    const char* name;
    hipEvent_t begin, end;
  };
  std::vector<Span> spans;
  uint32_t err_ops_saved = 0;  // err_ops of the eager stream while a graph is recorded
  std::vector<struct fo_graph*> graveyard;  // graphs freed while recording, destroyed when it ends
  std::unordered_set<struct fo_graph*> graphs;  // live graphs recorded on this runtime
  // FO_EAGER=1 in the environment when the runtime is created: nothing is deferred (zero fills run
  // at allocation, casts, map chains and broadcasts run when issued), the reference check for the
  // deferred forms.
  bool eager = false;
};

// A recorded op stream (fo_graph_begin .. fo_graph_end), launched as one HIP graph.
struct fo_graph {
  fo_runtime* rt = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::shared_ptr<fo_graph_mem> mem;
  uint32_t err_ops = 0;  // device error checks its launches owe the next synchronize
};

struct fo_buffer {
  void* ptr = nullptr;
  uint64_t bytes = 0;     // the size asked for
  uint64_t capacity = 0;  // the block's size (the pool's size class)
  int device = 0;
  std::shared_ptr<fo_pool> pool;
  // Zero-filled as allocated (Backend::zeroed), with the fill deferred to the buffer's first use:
  // an op that overwrites every byte drops it, any other use launches it first.
  bool zero_pending = false;
  // An exact widening cast into this buffer recorded but not yet run (the runtime's pending
  // widens): a read runs it first.
  // Read without the records' lock (a fast check before taking it), so atomic.
  std::atomic<bool> widen_pending{false};
  // Freed by its owner while a pending widen still reads it (the source of that widen): the block
  // stays until no widen record names it, then goes the way a free at retirement time would have
  // sent it (retired_in: the recording open then, if any).
  bool retired = false;
  std::shared_ptr<fo_graph_mem> retired_in;
  // Born while a graph was recorded: the block belongs to that recording's memory, not to the
  // pool, and outlives this buffer while the graph lives.
  std::shared_ptr<fo_graph_mem> graph_mem;
};

namespace fo {

struct InvalidArg : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct OomError : std::runtime_error {
  using std::runtime_error::runtime_error;
};
struct Unsupported : std::runtime_error {
  using std::runtime_error::runtime_error;
};

#define FO_HIP(call)                                                                              \
  do {                                                                                            \
    hipError_t _e = (call);                                                                       \
    if (_e != hipSuccess)                                                                         \
      throw ::fo::HipError(std::string(#call) + " failed: " + hipGetErrorString(_e));            \
  } while (0)

inline void require(bool cond, const std::string& what) {
  if (!cond) throw InvalidArg(what);
}

inline int64_t dtype_bytes(fo_dtype t) {
  switch (t) {
    case FO_I8:
    case FO_U8:
    case FO_F8E4M3:
    case FO_F8E5M2:
      return 1;
    case FO_I16:
    case FO_BF16:
      return 2;
    case FO_I32:
    case FO_F32:
      return 4;
    case FO_I4:
    case FO_F4E2M1:
      throw InvalidArg("4-bit (nibble-packed) elements are taken by map, contraction and transpose only");
  }
  throw InvalidArg("unknown dtype");
}

inline bool is_nibble(fo_dtype t) { return t == FO_I4 || t == FO_F4E2M1; }

// Bytes that hold n elements (a 4-bit stream packs two per byte).
inline uint64_t span_bytes(fo_dtype t, uint64_t n) { return is_nibble(t) ? (n + 1) / 2 : n * (uint64_t)dtype_bytes(t); }

// Host-side copy of wheels into the by-value kernel descriptor.
template <int NMEM>
Wheels<NMEM> to_desc(const std::vector<mapping::Wheel>& ws, const int (&mem)[NMEM]) {
  Wheels<NMEM> d{};
  require((int)ws.size() <= kMaxWheels, "mapping resolves to more than " + std::to_string(kMaxWheels) + " wheels");
  d.n = (int)ws.size();
  for (int i = 0; i < d.n; ++i) {
    require(ws[i].size < (1ll << 31), "wheel too large for 32-bit addressing");
    d.size[i] = (uint32_t)ws[i].size;
    d.live[i] = (uint32_t)ws[i].live;
    d.div[i] = FastDiv((uint32_t)ws[i].size);
    for (int k = 0; k < NMEM; ++k) d.stride[k][i] = ws[i].stride[mem[k]];
  }
  return d;
}

// ---- launchers (one per kernel family) ----------------------------------------------------------

// Transpose: dst[dst_base + p] = src[src_base + off(p)] for live p < count.
// The f32 relayout of bf16 data standing for its exact widen, when the chunked copy applies (every
// dst run a multiple of four elements, contiguous in src); false when it does not (k_storage.hip).
bool launch_relayout_widen(hipStream_t s, float* dst, const uint16_t* src, int64_t dst_base, int64_t src_base,
                           int64_t count, const Wheels<1>& w);
void launch_relayout(hipStream_t s, void* dst, const void* src, int64_t elem_bytes, int64_t dst_base, int64_t src_base,
                     int64_t count, const Wheels<1>& w);
// A chain of full-view transposes as one gather. Step k writes its positions p < count (a live
// digit walk of its wheels) into a fresh zeroed storage from src_base + off(p) of the previous one.
// The kernel covers positions [0, total) of the last storage; those the last step does not write
// are zeroed when `zero_unwritten` (the last storage is itself a fresh intermediate), else kept.
constexpr int kMaxChain = 6;
struct ChainStep {
  Wheels<1> w;
  int64_t src_base;
  uint32_t count;
};
struct Chain {
  int32_t n = 0;
  int32_t zero_unwritten = 0;
  uint32_t total = 0;
  ChainStep step[kMaxChain];
};
void launch_relayout_chain(hipStream_t s, void* dst, const void* src, int64_t elem_bytes, const Chain& c);
// The chain over 4-bit elements (two per byte); final position p goes to dst element dst_base + p,
// and a byte's nibble the chain does not write keeps its value.
void launch_relayout_chain_nibble(hipStream_t s, void* dst, const void* src, const Chain& c, uint64_t dst_base);
// Gather: dst[off_d(p*slots + r)] = src[off_s(p*axis + index[r] / div)]; bad indices skipped, *flag = 1.
// `*_slot_wheels`: how many innermost wheels of each list belong to the slot / axis part (the
// payload's wheels follow), for the 16-byte payload path.
void launch_gather(hipStream_t s, void* dst, const void* src, const int32_t* idx, int64_t elem_bytes,
                   int64_t payload, int64_t slots, int64_t axis_size, int32_t div, const Wheels<1>& ws,
                   const Wheels<1>& wd, int ws_slot_wheels, int wd_slot_wheels, int32_t* flag);
// Scatter: dst[off_d(p*axis + index[k] / div)] = src[off_s(p*keys + k)], the last key k winning a
// repeated index (win: axis_size i32 set to -1 beforehand); bad indices skipped, *flag = 1.
void launch_scatter(hipStream_t s, void* dst, const void* src, const int32_t* idx, int64_t elem_bytes,
                    int64_t payload, int64_t keys, int64_t axis_size, int32_t div, const Wheels<1>& ws,
                    const Wheels<1>& wd, int ws_slot_wheels, int wd_slot_wheels, uint64_t* win, uint32_t gen,
                    int32_t* flag);
// Transmute: dst live rank k <- src live rank k; dst padding zeroed.
void launch_transmute(hipStream_t s, void* dst, const void* src, int64_t elem_bytes, int64_t dst_count,
                      const Wheels<1>& dst_self, const Wheels<1>& src_self);

void launch_map(hipStream_t s, void* dst, fo_dtype dst_t, const void* src, fo_dtype src_t, uint64_t n, const fo_op& op);
// i4 stream of `nbytes` -> 2 * nbytes i8 elements; i32 accumulators -> i4 stream (n even)
void launch_unpack_i4(hipStream_t s, int8_t* dst, const void* src, uint64_t nbytes);
void launch_pack_i4(hipStream_t s, void* dst, const int32_t* src, uint64_t n);
void launch_zip(hipStream_t s, void* dst, fo_dtype dst_t, const void* a, const void* b, fo_dtype in_t, uint64_t n,
                const fo_op& op);
// *flag = 1 when a tag byte is above 15 (not an execution id).
// zip_with (f32 out) and map (f32 or bf16 out) over f32 inputs that stand for deferred casts
// (k_vector.hip). An input's read code: 4 = f32 data as is; 2 = the bf16 source of a deferred exact
// widen; kReadViaBf16 = the f32 source of a deferred bf16 narrow that a deferred widen reads,
// rounded through bf16 on load.
constexpr int kReadViaBf16 = 5;
// Deferred f32 -> f32 maps a zip input is read through, applied in order after the load (and the
// widen of bf16 data) and before the bf16 round trip of kReadViaBf16.
struct PreOps {
  int32_t n = 0;
  fo_op op[3] = {};
};
void launch_zip_widened(hipStream_t s, void* dst, fo_dtype dst_t, const void* a, int a_code, const PreOps& a_pre,
                        const void* b, int b_code, const PreOps& b_pre, uint64_t n, const fo_op& op);
// zip_with over f32 inputs (f32 out) given as (data, read code, div, mod): element i of an input is
// element (i / div) % mod of its data (mod 0: no wrap), a broadcast recorded by a transpose.
void launch_zip_bcast(hipStream_t s, void* dst, const void* a, int a_code, uint32_t a_div, uint32_t a_mod,
                      const PreOps& a_pre, const void* b, int b_code, uint32_t b_div, uint32_t b_mod,
                      const PreOps& b_pre, uint64_t n, const fo_op& op);
void launch_map_widened(hipStream_t s, void* dst, fo_dtype dst_t, const void* src, int src_code, uint64_t n,
                        const fo_op& op);
void launch_zip3_slots(hipStream_t s, void* dst, const void* data, const void* port, const uint8_t* tag, fo_dtype t,
                       uint64_t n, const fo_slots& slots, int32_t* flag);
void launch_branch_tag(hipStream_t s, uint8_t* dst, const void* src, fo_dtype t, uint64_t n, const fo_cmp* cmps);

// Reduce over a plan: out wheels (memory strides into src) and residue wheels.
// An f32 reduce whose source is bf16 data standing for its exact widen, or (via_bf16) f32 data
// standing for the widen of its deferred bf16 narrow (k_storage.hip).
void launch_reduce_widened(hipStream_t s, void* dst, const void* src, bool via_bf16, int64_t src_len,
                           int64_t out_count, const Wheels<1>& ow, const Wheels<1>& rw, int op, uint32_t identity);
void launch_reduce(hipStream_t s, void* dst, const void* src, fo_dtype t, int64_t src_len, int64_t out_count,
                   const Wheels<1>& out_w, const Wheels<1>& res_w, int op, uint32_t identity);

// A reduce whose output cells are contiguous, split over residue chunks with partials in scratch
// (4-byte regroupable folds only). nchunks == 0: the layout does not qualify.
struct ReduceSplit {
  int64_t nchunks = 0, chunk_len = 0;
  uint64_t scratch_bytes = 0;
};
ReduceSplit plan_reduce_split(fo_dtype t, int op, const void* src, int64_t src_len, int64_t out_count,
                              const Wheels<1>& out_w, const Wheels<1>& res_w);
void launch_reduce_split(hipStream_t s, void* dst, const void* src, fo_dtype t, int64_t out_count,
                         const Wheels<1>& out_w, const Wheels<1>& res_w, int op, uint32_t identity,
                         const ReduceSplit& plan, void* scratch);

// Generic contraction: out wheels / residue wheels with strides into (lhs, rhs).
// Batched dot products (k_contract_dot): every out wheel reads both operands, the residue K
// contiguous elements in both; vec: every row start 16-byte aligned. False for a type pair it does
// not take.
// k_storage.hip: an affine contraction (one row, column, batch and contracted wheel each; A(m, k) =
// a_batch*b + lda*m + sa*k, B(n, k) = b_batch*b + ldb*n + sb*k) of f32 -> f32, i32 -> i32, bf16 ->
// f32 / bf16 or i8 -> i32 / i8, each cell the serial fold in k order (bit-exact); false when the
// shape or types do not fit the kernel.
struct GemmDesc;
bool launch_contraction_simt(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t, fo_dtype out_t,
                             const GemmDesc& d, int64_t sa, int64_t sb);
bool launch_contraction_dot(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t, fo_dtype out_t,
                            int64_t n, const Wheels<2>& ow, int64_t K, bool vec);
void launch_contraction_generic(hipStream_t s, void* out, const void* lhs, const void* rhs, fo_dtype in_t,
                                fo_dtype out_t, int64_t lhs_len, int64_t rhs_len, int64_t out_count,
                                const Wheels<2>& out_w, const Wheels<2>& res_w);

// MFMA GEMM for a contraction shaped C[m, n] = sum_k A[m, k] B[n, k] with k contiguous in both.
struct GemmDesc {
  int64_t M = 0, N = 0, K = 0;
  int64_t batch = 1;
  // element offsets: A(m,k) = a_batch*b + lda*m + k ; B(n,k) = b_batch*b + ldb*n + k ;
  // C(m,n) = c_batch*b + ldc_m*m + ldc_n*n.
  int64_t a_batch = 0, b_batch = 0, c_batch = 0;
  int64_t lda = 0, ldb = 0, ldc_m = 0, ldc_n = 1;
};
// in_t FO_BF16 -> out FO_BF16 / FO_F32; in_t FO_I8 -> out FO_I8 / FO_I32.
// k_gemv.hip: one bf16 vector x [K] against rows w[n * ldw + k]; out[n * ldo] (f32 or bf16) is the
// serial fold of each cell in k order (the emulator's contraction_in, bit-exact).
bool gemv_supported(fo_dtype in_t, fo_dtype out_t, const void* x, const void* w, int64_t N, int64_t K,
                    int64_t ldw);
// x_f32: x is f32 data standing for the widen of its deferred bf16 narrow, rounded as it is staged
// (gemv_takes_f32_x(K) says whether the kernel for K has that form).
bool gemv_takes_f32_x(int64_t K);
void launch_gemv(hipStream_t s, void* out, const void* x, const void* w, fo_dtype in_t, fo_dtype out_t, int64_t N,
                 int64_t K, int64_t ldw, int64_t ldo, bool x_f32 = false);
void launch_gemm(hipStream_t s, void* c, const void* a, const void* b, fo_dtype in_t, fo_dtype out_t,
                 const GemmDesc& d);
bool gemm_supported(fo_dtype in_t, fo_dtype out_t);
bool gemm_aligned(const void* a, const void* b, fo_dtype in_t, const GemmDesc& d);

// MFMA contraction over wheel-decoded rows / columns / batch cells (k_gemm_wheels.hip):
// A(b, m, k) = off_a(b) + off_a(m) + k, B(b, n, k) = off_b(b) + off_b(n) + k,
// C(b, m, n) = off_c(b) + off_c(m) + off_c(n); mw strides {A, C}, nw {B, C}, bw {A, B, C}; wheels
// hold live digits only. `elem_align`: the gcd of the operand strides and K (in elements).
bool gemm_wheels_supported(fo_dtype in_t, fo_dtype out_t, int64_t K, int64_t elem_align);
void launch_gemm_wheels(hipStream_t s, void* c, const void* a, const void* b, fo_dtype in_t, fo_dtype out_t,
                        int64_t M, int64_t N, int64_t K, int64_t batches, const Wheels<2>& mw, const Wheels<2>& nw,
                        const Wheels<3>& bw);
// Zeroes `bytes` bytes at a 16-byte aligned device address (a fill kernel, not hipMemsetAsync).
void launch_zero(hipStream_t s, void* p, uint64_t bytes);

void launch_w8a8(hipStream_t s, uint16_t* out, int32_t* acc_out, const int8_t* a, const int8_t* w, const float* scale,
                 int64_t m, int64_t n, int64_t k);
void launch_rmsnorm_softmax(hipStream_t s, uint16_t* out, const uint16_t* x, const uint16_t* gain, int64_t rows,
                            int64_t cols, float eps);
void launch_attention_prefill(hipStream_t s, uint16_t* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const float* row_max, int64_t batch, int64_t heads, int64_t seq, int64_t head_dim,
                              float sqrt_d, int causal);
void launch_mlp(hipStream_t s, int32_t* pred, uint16_t* logits, const uint16_t* x, const uint16_t* w1,
                const uint16_t* b1, const uint16_t* w2, const uint16_t* b2, int64_t batch, int64_t in_f,
                int64_t hidden, int64_t out_f);

}  // namespace fo
