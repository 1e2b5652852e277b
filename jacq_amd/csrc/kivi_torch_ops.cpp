// Torch custom ops over libjacq_kivi.so, built with hipcc for gfx950
// (libjacq_kivi_torch.so, namespace torch.ops.jacq_kivi):
//
//  * the reference's vLLM op surface -- the seven ops the patched
//    csrc/torch_bindings.cpp registers (integrations/vllm_kivi/
//    source_patch.py:2797-2870), with the fail-closed validators of
//    KIVI_BINDING_SOURCE (:673-1495): same schemas, argument meaning, checks
//    and error texts.  Each op calls the v1 symbol of include/jacq_kivi.h that
//    the reference op calls;
//  * a "<op>_check" twin of every op: the same validators without the two
//    that need device tensors (GPU residency and the device's architecture),
//    registered for every backend, so the rejection table runs on a CPU host;
//  * ResidualSlots, the decode lane's residual-slot allocator (source_patch.py
//    :3047-3098): a request keeps one residual-scratch slot for its lifetime,
//    finished and vanished requests give theirs back, and running out after
//    the last reclaim raises NotImplementedError.
//
// The device check reads the architecture of the device the tensors live on
// (hipGetDeviceProperties().gcnArchName, feature suffixes ignored) and
// accepts gfx950 only, where the reference accepts sm_80 / sm_89 (:719-742).

#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <hip/hip_runtime_api.h>
#include <torch/custom_class.h>
#include <torch/library.h>

#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <optional>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include "jacq_kivi.h"

namespace jacq_ops {

// The v1 lane (source_patch.py:660-671).
constexpr int64_t kHeads = 40, kKvHeads = 8;            // global geometry
constexpr int64_t kLocalHeads = 20, kLocalKvHeads = 4;  // TP=2 local rank
constexpr int64_t kHeadDim = 128, kPacked = kHeadDim / 2, kGroupsPerHead = kHeadDim / 32;
constexpr int64_t kTablePages = 124, kPageTokens = 32, kResidual = 128;
constexpr int64_t kScratchRows = kResidual + kPageTokens;  // 160
constexpr int64_t kMaxQueries = 160;
constexpr int64_t kMaxSeqLen = kTablePages * kPageTokens + kResidual;  // 4096

// Launch: every check, then the kernel.  Check: the same checks minus GPU
// residency and the device architecture; nothing is launched.
enum class Mode { Launch, Check };

const char* dtype_label(at::ScalarType s) {
  switch (s) {
    case at::kHalf: return "fp16";
    case at::kFloat: return "fp32";
    case at::kInt: return "int32";
    case at::kLong: return "int64";
    case at::kByte: return "uint8";
    default: return "?";
  }
}

template <Mode M>
void placed(const at::Tensor& t, const char* name) {
  if (M == Mode::Launch) TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous for jac_launch");
}

void dtype_is(const at::Tensor& t, at::ScalarType s, const char* name) {
  TORCH_CHECK(t.scalar_type() == s, name, " must be ", dtype_label(s));
}

void shape_is(const at::Tensor& t, std::initializer_list<int64_t> dims, const char* name) {
  TORCH_CHECK(t.dim() == (int64_t)dims.size(), name, " rank mismatch for the KIVI DSL ABI");
  int64_t axis = 0;
  for (int64_t want : dims) {
    TORCH_CHECK(t.size(axis) == want, name, " dim ", axis, " must be ", want,
                " for the KIVI DSL ABI, got ", t.size(axis));
    ++axis;
  }
}

// Pages of the table a length needs (source_patch.py:692-707): whole
// 32-token groups aged past the 128-token residual, 0 through 159 tokens.
void table_covers(const at::Tensor& t, const char* name, int64_t seq_len) {
  TORCH_CHECK(t.dim() == 1, name, " rank mismatch for the KIVI DSL ABI");
  TORCH_CHECK(seq_len >= 1 && seq_len <= kMaxSeqLen,
              "SEQ_LEN must be in [1, 4096] for KIVI BLOCK_TABLE validation");
  const int64_t pages = seq_len > kResidual ? (seq_len - kResidual) / kPageTokens : 0;
  TORCH_CHECK(t.size(0) >= pages, name, " dim 0 must be at least ", pages,
              " for the KIVI DSL ABI, got ", t.size(0));
}

bool is_local(int64_t nh, int64_t nkv) { return nh == kLocalHeads && nkv == kLocalKvHeads; }

void geometry_is_supported(int64_t nh, int64_t nkv, const char* op) {
  TORCH_CHECK((nh == kHeads && nkv == kKvHeads) || is_local(nh, nkv), op,
              " supports global NH/NKV 40/8 or TP=2 local-rank NH/NKV 20/4; got NH=", nh,
              " NKV=", nkv);
}

// One device for every tensor, and that device a gfx950.
template <Mode M>
void device_is_validated(std::initializer_list<const at::Tensor*> ts, const char* op) {
  if (M == Mode::Check) return;
  TORCH_CHECK(ts.size() > 0, op, " requires at least one tensor");
  const c10::Device dev = (*ts.begin())->device();
  TORCH_CHECK(dev.is_cuda(), op, " tensors must be bound to a GPU device, got ", dev);
  for (const at::Tensor* t : ts)
    TORCH_CHECK(t->device() == dev, op, " tensors must all live on one GPU device; got ",
                t->device(), " alongside ", dev);
  hipDeviceProp_t prop{};
  const hipError_t e = hipGetDeviceProperties(&prop, dev.index());
  TORCH_CHECK(e == hipSuccess, op, ": hipGetDeviceProperties failed for GPU device ",
              (int)dev.index(), ": ", hipGetErrorString(e));
  std::string arch(prop.gcnArchName);
  arch = arch.substr(0, arch.find(':'));
  TORCH_CHECK(arch == "gfx950", op, ": actual GPU device ", (int)dev.index(), " reports ",
              prop.gcnArchName, ", outside the validated set gfx950 (MI355X); refusing to launch");
}

hipStream_t stream_of(const at::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

template <class T>
T* ptr(const at::Tensor& t) {
  return reinterpret_cast<T*>(t.data_ptr());
}

// The eight cache tensors every op takes, in the reference's argument order.
struct Pool {
  const at::Tensor& kc;
  const at::Tensor& ks;
  const at::Tensor& kz;
  const at::Tensor& vc;
  const at::Tensor& vs;
  const at::Tensor& vz;
  const at::Tensor& kscr;
  const at::Tensor& vscr;

  template <Mode M>
  void placed_all() const {
    placed<M>(kc, "K_CODE_PAGES");
    placed<M>(ks, "K_SCALE_PAGES");
    placed<M>(kz, "K_ZERO_PAGES");
    placed<M>(vc, "V_CODE_PAGES");
    placed<M>(vs, "V_SCALE_PAGES");
    placed<M>(vz, "V_ZERO_PAGES");
    placed<M>(kscr, "K_RESIDUAL_SCRATCH");
    placed<M>(vscr, "V_RESIDUAL_SCRATCH");
  }
  void dtypes() const {
    dtype_is(kc, at::kByte, "K_CODE_PAGES");
    dtype_is(vc, at::kByte, "V_CODE_PAGES");
    dtype_is(ks, at::kHalf, "K_SCALE_PAGES");
    dtype_is(kz, at::kHalf, "K_ZERO_PAGES");
    dtype_is(vs, at::kHalf, "V_SCALE_PAGES");
    dtype_is(vz, at::kHalf, "V_ZERO_PAGES");
    dtype_is(kscr, at::kHalf, "K_RESIDUAL_SCRATCH");
    dtype_is(vscr, at::kHalf, "V_RESIDUAL_SCRATCH");
  }
  int64_t kv_heads() const {
    TORCH_CHECK(kc.dim() >= 2, "K_CODE_PAGES must expose NKV at dim 1");
    return kc.size(1);
  }
  // The leading dimension is the pool's page capacity, read from the tensor
  // itself; the table width and the length ceiling stay tied to 124 pages.
  int64_t pages() const { return kc.size(0); }
  void positive_capacity() const {
    TORCH_CHECK(pages() > 0, "K_CODE_PAGES dim 0 (page storage capacity) must be positive");
  }
  void shapes(int64_t nkv) const {
    const int64_t n = pages();
    shape_is(kc, {n, nkv, kPageTokens, kPacked}, "K_CODE_PAGES");
    shape_is(ks, {n, nkv, kHeadDim}, "K_SCALE_PAGES");
    shape_is(kz, {n, nkv, kHeadDim}, "K_ZERO_PAGES");
    shape_is(vc, {n, nkv, kPageTokens, kPacked}, "V_CODE_PAGES");
    shape_is(vs, {n, nkv, kPageTokens, kGroupsPerHead}, "V_SCALE_PAGES");
    shape_is(vz, {n, nkv, kPageTokens, kGroupsPerHead}, "V_ZERO_PAGES");
    shape_is(kscr, {nkv, kScratchRows, kHeadDim}, "K_RESIDUAL_SCRATCH");
    shape_is(vscr, {nkv, kScratchRows, kHeadDim}, "V_RESIDUAL_SCRATCH");
  }
};

// ---- decodes ----

// source_patch.py:768-869 -> jac_launch / jac_launch_tp2_local
template <Mode M>
void decode_dsl(const at::Tensor& q, const at::Tensor& bt, const at::Tensor& kc,
                const at::Tensor& ks, const at::Tensor& kz, const at::Tensor& vc,
                const at::Tensor& vs, const at::Tensor& vz, const at::Tensor& kscr,
                const at::Tensor& vscr, int64_t seq_len, const at::Tensor& out) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  placed<M>(q, "Q");
  placed<M>(bt, "BLOCK_TABLE");
  p.placed_all<M>();
  placed<M>(out, "O");
  dtype_is(q, at::kHalf, "Q");
  dtype_is(bt, at::kInt, "BLOCK_TABLE");
  p.dtypes();
  dtype_is(out, at::kFloat, "O");
  const int64_t nh = q.size(0), nkv = p.kv_heads();
  geometry_is_supported(nh, nkv, "kivi_decode_dsl");
  p.positive_capacity();
  shape_is(q, {nh, kHeadDim}, "Q");
  table_covers(bt, "BLOCK_TABLE", seq_len);
  p.shapes(nkv);
  shape_is(out, {nh, kHeadDim}, "O");
  TORCH_CHECK(seq_len >= 1 && seq_len <= kMaxSeqLen,
              "SEQ_LEN must be in [1, 4096] for the KIVI DSL ABI");
  device_is_validated<M>({&q, &bt, &kc, &ks, &kz, &vc, &vs, &vz, &kscr, &vscr, &out},
                         "kivi_decode_dsl");
  if (M == Mode::Check) return;
  (is_local(nh, nkv) ? jac_launch_tp2_local : jac_launch)(
      ptr<const jacq_half_t>(q), ptr<const int32_t>(bt), ptr<const uint8_t>(kc),
      ptr<const jacq_half_t>(ks), ptr<const jacq_half_t>(kz), ptr<const uint8_t>(vc),
      ptr<const jacq_half_t>(vs), ptr<const jacq_half_t>(vz), ptr<const jacq_half_t>(kscr),
      ptr<const jacq_half_t>(vscr), (int)seq_len, ptr<float>(out), stream_of(q));
}

// source_patch.py:872-971 -> jac_launch_sparse_retained(_tp2_local)
template <Mode M>
void decode_sparse_retained_dsl(const at::Tensor& q, const at::Tensor& rbt,
                                const at::Tensor& kc, const at::Tensor& ks,
                                const at::Tensor& kz, const at::Tensor& vc,
                                const at::Tensor& vs, const at::Tensor& vz,
                                const at::Tensor& kscr, const at::Tensor& vscr, int64_t seq_len,
                                int64_t retained, const at::Tensor& out) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  const char* op = "kivi_decode_sparse_retained_dsl";
  placed<M>(q, "Q");
  placed<M>(rbt, "RETAINED_BLOCK_TABLE");
  p.placed_all<M>();
  placed<M>(out, "O");
  dtype_is(q, at::kHalf, "Q");
  dtype_is(rbt, at::kInt, "RETAINED_BLOCK_TABLE");
  p.dtypes();
  dtype_is(out, at::kFloat, "O");
  const int64_t nh = q.size(0), nkv = p.kv_heads();
  geometry_is_supported(nh, nkv, op);
  p.positive_capacity();
  shape_is(q, {nh, kHeadDim}, "Q");
  shape_is(rbt, {kTablePages}, "RETAINED_BLOCK_TABLE");
  p.shapes(nkv);
  shape_is(out, {nh, kHeadDim}, "O");
  TORCH_CHECK(seq_len >= 1 && seq_len <= kMaxSeqLen,
              "SEQ_LEN must be in [1, 4096] for the KIVI sparse-retained DSL ABI");
  TORCH_CHECK(retained >= 0 && retained <= kTablePages,
              "NUM_RETAINED_PAGES must be in [0, OLD_BLOCKS]");
  TORCH_CHECK(retained <= p.pages(),
              "NUM_RETAINED_PAGES cannot exceed physical page storage capacity");
  device_is_validated<M>({&q, &rbt, &kc, &ks, &kz, &vc, &vs, &vz, &kscr, &vscr, &out}, op);
  if (M == Mode::Check) return;
  (is_local(nh, nkv) ? jac_launch_sparse_retained_tp2_local : jac_launch_sparse_retained)(
      ptr<const jacq_half_t>(q), ptr<const int32_t>(rbt), ptr<const uint8_t>(kc),
      ptr<const jacq_half_t>(ks), ptr<const jacq_half_t>(kz), ptr<const uint8_t>(vc),
      ptr<const jacq_half_t>(vs), ptr<const jacq_half_t>(vz), ptr<const jacq_half_t>(kscr),
      ptr<const jacq_half_t>(vscr), (int)seq_len, (int)retained, ptr<float>(out), stream_of(q));
}

// source_patch.py:1268-1386 -> jac_launch_batched(_tp2_local): up to 160
// causal queries of one sequence.  The lengths are read back to the host so
// a bad one stops the call before launch, as the reference does (:1352-1360).
template <Mode M>
void decode_batched_dsl(const at::Tensor& q, const at::Tensor& seq_lens, const at::Tensor& bt,
                        const at::Tensor& kc, const at::Tensor& ks, const at::Tensor& kz,
                        const at::Tensor& vc, const at::Tensor& vs, const at::Tensor& vz,
                        const at::Tensor& kscr, const at::Tensor& vscr, int64_t num_queries,
                        const at::Tensor& out) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  const char* op = "kivi_decode_batched_dsl";
  placed<M>(q, "Q");
  placed<M>(seq_lens, "SEQ_LENS");
  placed<M>(bt, "BLOCK_TABLE");
  p.placed_all<M>();
  placed<M>(out, "O");
  dtype_is(q, at::kHalf, "Q");
  dtype_is(seq_lens, at::kInt, "SEQ_LENS");
  dtype_is(bt, at::kInt, "BLOCK_TABLE");
  p.dtypes();
  dtype_is(out, at::kFloat, "O");
  TORCH_CHECK(q.dim() == 3, "Q rank mismatch for the batched KIVI DSL decode ABI");
  const int64_t nh = q.size(1), nkv = p.kv_heads();
  geometry_is_supported(nh, nkv, op);
  p.positive_capacity();
  TORCH_CHECK(num_queries >= 1 && num_queries <= kMaxQueries,
              "NUM_QUERIES must be in [1, MAX_QUERIES] for the batched KIVI DSL decode ABI");
  shape_is(q, {num_queries, nh, kHeadDim}, "Q");
  shape_is(seq_lens, {num_queries}, "SEQ_LENS");
  p.shapes(nkv);
  shape_is(out, {num_queries, nh, kHeadDim}, "O");
  const at::Tensor lens = seq_lens.to(at::kCPU);
  const int32_t* lv = lens.data_ptr<int32_t>();
  for (int64_t i = 0; i < num_queries; ++i) {
    TORCH_CHECK(lv[i] >= 1 && lv[i] <= kMaxSeqLen, "SEQ_LENS[", i,
                "] must be in [1, 4096] for the batched KIVI DSL decode ABI, got ", lv[i]);
    table_covers(bt, "BLOCK_TABLE", lv[i]);
  }
  device_is_validated<M>({&q, &seq_lens, &bt, &kc, &ks, &kz, &vc, &vs, &vz, &kscr, &vscr, &out},
                         op);
  if (M == Mode::Check) return;
  (is_local(nh, nkv) ? jac_launch_batched_tp2_local : jac_launch_batched)(
      ptr<const jacq_half_t>(q), ptr<const int32_t>(seq_lens), ptr<const int32_t>(bt),
      ptr<const uint8_t>(kc), ptr<const jacq_half_t>(ks), ptr<const jacq_half_t>(kz),
      ptr<const uint8_t>(vc), ptr<const jacq_half_t>(vs), ptr<const jacq_half_t>(vz),
      ptr<const jacq_half_t>(kscr), ptr<const jacq_half_t>(vscr), (int)num_queries,
      ptr<float>(out), stream_of(q));
}

// ---- writers ----

// Which writer entry an op reaches and what it accepts.
enum class Writer {
  Hand,        // kivi_cache_write(_batched)_launch: global or TP=2 local kv heads
  Generated,   // jac_launch_cache_write(_batched): global geometry only
};

// The checks the four writer ops share (source_patch.py:975-1078,
// 1085-1180, 1185-1262, 1392-1495).  single: a one-token writer (NEW_K/NEW_V
// [NKV, HD], one SLOT_MAPPING entry, `start` the length after the write);
// otherwise num_new tokens appended at length `start`.
template <Mode M>
int64_t writer_checks(const char* op, Writer which, const Pool& p, const at::Tensor& nk,
                      const at::Tensor& nv, const at::Tensor& slots, const at::Tensor& bt,
                      bool single, int64_t start, int64_t num_new) {
  p.placed_all<M>();
  placed<M>(nk, "NEW_K");
  placed<M>(nv, "NEW_V");
  placed<M>(slots, "SLOT_MAPPING");
  placed<M>(bt, "BLOCK_TABLE");
  p.dtypes();
  dtype_is(nk, at::kHalf, "NEW_K");
  dtype_is(nv, at::kHalf, "NEW_V");
  dtype_is(slots, at::kLong, "SLOT_MAPPING");
  dtype_is(bt, at::kInt, "BLOCK_TABLE");
  int64_t nkv = kKvHeads;
  if (which == Writer::Hand) {
    nkv = p.kv_heads();
    geometry_is_supported(nkv == kKvHeads ? kHeads : kLocalHeads, nkv, op);
  }
  p.positive_capacity();
  if (!single)
    TORCH_CHECK(num_new >= 1 && num_new <= kScratchRows,
                "NUM_NEW must be in [1, RESIDUAL_SCRATCH] -- callers must pre-split a prefill "
                "chunk into sub-chunks via plan_batched_write before calling this op");
  p.shapes(nkv);
  if (single) {
    shape_is(nk, {nkv, kHeadDim}, "NEW_K");
    shape_is(nv, {nkv, kHeadDim}, "NEW_V");
    table_covers(bt, "BLOCK_TABLE", start);
    TORCH_CHECK(slots.numel() == 1,
                "SLOT_MAPPING must contain exactly one decode token in the first KIVI DSL "
                "writer lane");
    TORCH_CHECK(start >= 1 && start <= kMaxSeqLen,
                "SEQ_LEN must be in [1, 4096] for the first KIVI DSL writer lane");
  } else {
    shape_is(nk, {num_new, nkv, kHeadDim}, "NEW_K");
    shape_is(nv, {num_new, nkv, kHeadDim}, "NEW_V");
    table_covers(bt, "BLOCK_TABLE", start + num_new);
    TORCH_CHECK(slots.numel() == num_new, "SLOT_MAPPING must contain exactly NUM_NEW entries for ",
                which == Writer::Hand ? "the batched KIVI DSL writer" : op);
    TORCH_CHECK(start >= 0 && start + num_new <= kMaxSeqLen,
                "START_SEQ_LEN + NUM_NEW must be in [0, 4096] for ",
                which == Writer::Hand ? "the batched KIVI DSL writer lane" : op);
  }
  device_is_validated<M>({&p.kc, &p.ks, &p.kz, &p.vc, &p.vs, &p.vz, &p.kscr, &p.vscr, &nk, &nv,
                          &slots, &bt},
                         op);
  return nkv;
}

#define JACQ_POOL_PTRS(p)                                                                    \
  ptr<uint8_t>(p.kc), ptr<jacq_half_t>(p.ks), ptr<jacq_half_t>(p.kz), ptr<uint8_t>(p.vc),    \
      ptr<jacq_half_t>(p.vs), ptr<jacq_half_t>(p.vz), ptr<jacq_half_t>(p.kscr),              \
      ptr<jacq_half_t>(p.vscr)

// source_patch.py:975-1078 -> kivi_cache_write_launch
template <Mode M>
void cache_write_dsl(const at::Tensor& kc, const at::Tensor& ks, const at::Tensor& kz,
                     const at::Tensor& vc, const at::Tensor& vs, const at::Tensor& vz,
                     const at::Tensor& kscr, const at::Tensor& vscr, const at::Tensor& nk,
                     const at::Tensor& nv, const at::Tensor& slots, const at::Tensor& bt,
                     int64_t seq_len) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  const int64_t nkv =
      writer_checks<M>("kivi_cache_write_dsl", Writer::Hand, p, nk, nv, slots, bt, true, seq_len, 0);
  if (M == Mode::Check) return;
  kivi_cache_write_launch(JACQ_POOL_PTRS(p), ptr<const jacq_half_t>(nk),
                          ptr<const jacq_half_t>(nv), ptr<const int64_t>(slots),
                          ptr<const int32_t>(bt), (int)seq_len, (int)nkv, stream_of(kc));
}

// source_patch.py:1085-1180 -> jac_launch_cache_write (comparison op)
template <Mode M>
void cache_write_jac_dsl(const at::Tensor& kc, const at::Tensor& ks, const at::Tensor& kz,
                         const at::Tensor& vc, const at::Tensor& vs, const at::Tensor& vz,
                         const at::Tensor& kscr, const at::Tensor& vscr, const at::Tensor& nk,
                         const at::Tensor& nv, const at::Tensor& slots, const at::Tensor& bt,
                         int64_t seq_len) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  writer_checks<M>("kivi_cache_write_jac_dsl", Writer::Generated, p, nk, nv, slots, bt, true,
                   seq_len, 0);
  if (M == Mode::Check) return;
  jac_launch_cache_write(JACQ_POOL_PTRS(p), ptr<const jacq_half_t>(nk),
                         ptr<const jacq_half_t>(nv), ptr<const int32_t>(bt), (int)seq_len,
                         stream_of(kc));
}

// source_patch.py:1392-1495 -> kivi_cache_write_batched_launch
template <Mode M>
void cache_write_batched_dsl(const at::Tensor& kc, const at::Tensor& ks, const at::Tensor& kz,
                             const at::Tensor& vc, const at::Tensor& vs, const at::Tensor& vz,
                             const at::Tensor& kscr, const at::Tensor& vscr,
                             const at::Tensor& nk, const at::Tensor& nv, const at::Tensor& slots,
                             const at::Tensor& bt, int64_t start, int64_t num_new) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  const int64_t nkv = writer_checks<M>("kivi_cache_write_batched_dsl", Writer::Hand, p, nk, nv,
                                       slots, bt, false, start, num_new);
  if (M == Mode::Check) return;
  kivi_cache_write_batched_launch(JACQ_POOL_PTRS(p), ptr<const jacq_half_t>(nk),
                                  ptr<const jacq_half_t>(nv), ptr<const int64_t>(slots),
                                  ptr<const int32_t>(bt), (int)start, (int)num_new, (int)nkv,
                                  stream_of(kc));
}

// source_patch.py:1185-1262 -> jac_launch_cache_write_batched (comparison op)
template <Mode M>
void cache_write_batched_jac_dsl(const at::Tensor& kc, const at::Tensor& ks,
                                 const at::Tensor& kz, const at::Tensor& vc,
                                 const at::Tensor& vs, const at::Tensor& vz,
                                 const at::Tensor& kscr, const at::Tensor& vscr,
                                 const at::Tensor& nk, const at::Tensor& nv,
                                 const at::Tensor& slots, const at::Tensor& bt, int64_t start,
                                 int64_t num_new) {
  const Pool p{kc, ks, kz, vc, vs, vz, kscr, vscr};
  writer_checks<M>("kivi_cache_write_batched_jac_dsl", Writer::Generated, p, nk, nv, slots, bt,
                   false, start, num_new);
  if (M == Mode::Check) return;
  jac_launch_cache_write_batched(JACQ_POOL_PTRS(p), ptr<const jacq_half_t>(nk),
                                 ptr<const jacq_half_t>(nv), ptr<const int32_t>(bt), (int)start,
                                 (int)num_new, stream_of(kc));
}

#undef JACQ_POOL_PTRS

// ---- residual-slot allocator (source_patch.py:3047-3098) ----
//
// Slots index the per-request residual scratch.  A request keeps its slot
// from its first decode step to its end.  Each step: slots of finished
// requests go back to the free list; with the active set known, so do those
// of mapped requests no longer active; then every request of the step gets
// its slot, a new one from the free list (last freed first) or the next
// never-used index while fewer than max_seqs are mapped.  When neither is
// left, mapped requests absent from this step are reclaimed once more; if
// that frees nothing, the call raises NotImplementedError.  Reclaims walk the
// requests in the order they were first mapped, which fixes which slot a
// later request receives.  Used and free slots together are always
// 0 .. n-1 for the n slots ever handed out, so a new index never collides.
struct ResidualSlots : torch::CustomClassHolder {
  int64_t max_seqs;
  std::vector<std::pair<std::string, int64_t>> mapped;  // in first-mapped order
  std::vector<int64_t> free_list;

  explicit ResidualSlots(int64_t max) : max_seqs(max) {
    TORCH_CHECK(max >= 1, "ResidualSlots needs max_seqs >= 1, got ", max);
  }

  int64_t find(const std::string& id) const {
    for (size_t i = 0; i < mapped.size(); ++i)
      if (mapped[i].first == id) return (int64_t)i;
    return -1;
  }
  void release_at(size_t i) {
    free_list.push_back(mapped[i].second);
    mapped.erase(mapped.begin() + (std::ptrdiff_t)i);
  }
  // free every mapped request not in `keep`, in first-mapped order
  void release_absent(const std::unordered_set<std::string>& keep) {
    for (size_t i = 0; i < mapped.size();) {
      if (keep.count(mapped[i].first))
        ++i;
      else
        release_at(i);
    }
  }
  bool take(int64_t* slot) {
    if (!free_list.empty()) {
      *slot = free_list.back();
      free_list.pop_back();
      return true;
    }
    if ((int64_t)mapped.size() < max_seqs) {
      *slot = (int64_t)mapped.size();
      return true;
    }
    return false;
  }

  std::vector<int64_t> assign(std::vector<std::string> req_ids,
                              std::vector<std::string> finished,
                              std::optional<std::vector<std::string>> active) {
    for (const std::string& id : finished) {
      const int64_t i = find(id);
      if (i >= 0) release_at((size_t)i);
    }
    if (active) release_absent(std::unordered_set<std::string>(active->begin(), active->end()));
    const std::unordered_set<std::string> step(req_ids.begin(), req_ids.end());
    std::vector<int64_t> out;
    out.reserve(req_ids.size());
    for (const std::string& id : req_ids) {
      const int64_t i = find(id);
      if (i >= 0) {
        out.push_back(mapped[(size_t)i].second);
        continue;
      }
      int64_t slot = -1;
      if (!take(&slot)) {
        release_absent(step);  // pressure reclaim: nobody outside this step keeps a slot
        const bool got = take(&slot);
        TORCH_CHECK_NOT_IMPLEMENTED(
            got, "int4_kivi decode lane ran out of residual slots (max_seqs=", max_seqs,
            ") even after reclaim; ", mapped.size(),
            " distinct requests concurrently assigned and 0 free -- the serving engine's "
            "admission control (max_num_seqs) should make this unreachable, so a reclaim was "
            "missed");
      }
      mapped.emplace_back(id, slot);
      out.push_back(slot);
    }
    return out;
  }

  int64_t num_mapped() const { return (int64_t)mapped.size(); }
  int64_t num_free() const { return (int64_t)free_list.size(); }
  int64_t slot_of(std::string id) const {
    const int64_t i = find(id);
    return i < 0 ? -1 : mapped[(size_t)i].second;
  }
};

}  // namespace jacq_ops

// Schemas as the reference registers them (source_patch.py:2797-2870).
TORCH_LIBRARY(jacq_kivi, m) {
  static const char* kDecode =
      "(Tensor Q, Tensor BLOCK_TABLE, Tensor K_CODE_PAGES, Tensor K_SCALE_PAGES, "
      "Tensor K_ZERO_PAGES, Tensor V_CODE_PAGES, Tensor V_SCALE_PAGES, Tensor V_ZERO_PAGES, "
      "Tensor K_RESIDUAL_SCRATCH, Tensor V_RESIDUAL_SCRATCH, int SEQ_LEN, Tensor(a!) O) -> ()";
  static const char* kSparse =
      "(Tensor Q, Tensor RETAINED_BLOCK_TABLE, Tensor K_CODE_PAGES, Tensor K_SCALE_PAGES, "
      "Tensor K_ZERO_PAGES, Tensor V_CODE_PAGES, Tensor V_SCALE_PAGES, Tensor V_ZERO_PAGES, "
      "Tensor K_RESIDUAL_SCRATCH, Tensor V_RESIDUAL_SCRATCH, int SEQ_LEN, "
      "int NUM_RETAINED_PAGES, Tensor(a!) O) -> ()";
  static const char* kBatched =
      "(Tensor Q, Tensor SEQ_LENS, Tensor BLOCK_TABLE, Tensor K_CODE_PAGES, "
      "Tensor K_SCALE_PAGES, Tensor K_ZERO_PAGES, Tensor V_CODE_PAGES, Tensor V_SCALE_PAGES, "
      "Tensor V_ZERO_PAGES, Tensor K_RESIDUAL_SCRATCH, Tensor V_RESIDUAL_SCRATCH, "
      "int NUM_QUERIES, Tensor(a!) O) -> ()";
  static const char* kWrite =
      "(Tensor(a!) K_CODE_PAGES, Tensor(b!) K_SCALE_PAGES, Tensor(c!) K_ZERO_PAGES, "
      "Tensor(d!) V_CODE_PAGES, Tensor(e!) V_SCALE_PAGES, Tensor(f!) V_ZERO_PAGES, "
      "Tensor(g!) K_RESIDUAL_SCRATCH, Tensor(h!) V_RESIDUAL_SCRATCH, Tensor NEW_K, "
      "Tensor NEW_V, Tensor SLOT_MAPPING, Tensor BLOCK_TABLE, int SEQ_LEN) -> ()";
  static const char* kWriteBatched =
      "(Tensor(a!) K_CODE_PAGES, Tensor(b!) K_SCALE_PAGES, Tensor(c!) K_ZERO_PAGES, "
      "Tensor(d!) V_CODE_PAGES, Tensor(e!) V_SCALE_PAGES, Tensor(f!) V_ZERO_PAGES, "
      "Tensor(g!) K_RESIDUAL_SCRATCH, Tensor(h!) V_RESIDUAL_SCRATCH, Tensor NEW_K, "
      "Tensor NEW_V, Tensor SLOT_MAPPING, Tensor BLOCK_TABLE, int START_SEQ_LEN, "
      "int NUM_NEW) -> ()";
  const std::pair<const char*, const char*> ops[] = {
      {"kivi_decode_dsl", kDecode},
      {"kivi_decode_sparse_retained_dsl", kSparse},
      {"kivi_decode_batched_dsl", kBatched},
      {"kivi_cache_write_dsl", kWrite},
      {"kivi_cache_write_jac_dsl", kWrite},
      {"kivi_cache_write_batched_dsl", kWriteBatched},
      {"kivi_cache_write_batched_jac_dsl", kWriteBatched},
  };
  for (const auto& [name, args] : ops) {
    m.def((std::string(name) + args).c_str());
    m.def((std::string(name) + "_check" + args).c_str());
  }
  m.class_<jacq_ops::ResidualSlots>("ResidualSlots")
      .def(torch::init<int64_t>())
      .def("assign", &jacq_ops::ResidualSlots::assign)
      .def("num_mapped", &jacq_ops::ResidualSlots::num_mapped)
      .def("num_free", &jacq_ops::ResidualSlots::num_free)
      .def("slot_of", &jacq_ops::ResidualSlots::slot_of);
}

TORCH_LIBRARY_IMPL(jacq_kivi, CUDA, m) {
  using jacq_ops::Mode;
  m.impl("kivi_decode_dsl", &jacq_ops::decode_dsl<Mode::Launch>);
  m.impl("kivi_decode_sparse_retained_dsl", &jacq_ops::decode_sparse_retained_dsl<Mode::Launch>);
  m.impl("kivi_decode_batched_dsl", &jacq_ops::decode_batched_dsl<Mode::Launch>);
  m.impl("kivi_cache_write_dsl", &jacq_ops::cache_write_dsl<Mode::Launch>);
  m.impl("kivi_cache_write_jac_dsl", &jacq_ops::cache_write_jac_dsl<Mode::Launch>);
  m.impl("kivi_cache_write_batched_dsl", &jacq_ops::cache_write_batched_dsl<Mode::Launch>);
  m.impl("kivi_cache_write_batched_jac_dsl",
         &jacq_ops::cache_write_batched_jac_dsl<Mode::Launch>);
}

TORCH_LIBRARY_IMPL(jacq_kivi, CompositeExplicitAutograd, m) {
  using jacq_ops::Mode;
  m.impl("kivi_decode_dsl_check", &jacq_ops::decode_dsl<Mode::Check>);
  m.impl("kivi_decode_sparse_retained_dsl_check",
         &jacq_ops::decode_sparse_retained_dsl<Mode::Check>);
  m.impl("kivi_decode_batched_dsl_check", &jacq_ops::decode_batched_dsl<Mode::Check>);
  m.impl("kivi_cache_write_dsl_check", &jacq_ops::cache_write_dsl<Mode::Check>);
  m.impl("kivi_cache_write_jac_dsl_check", &jacq_ops::cache_write_jac_dsl<Mode::Check>);
  m.impl("kivi_cache_write_batched_dsl_check", &jacq_ops::cache_write_batched_dsl<Mode::Check>);
  m.impl("kivi_cache_write_batched_jac_dsl_check",
         &jacq_ops::cache_write_batched_jac_dsl<Mode::Check>);
}
