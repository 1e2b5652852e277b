// kivi_api.hip -- host side of libjacq_kivi.so: the C ABI of include/jacq_kivi.h.
//
// The v1 symbols keep the reference's launch contract (fixed geometry per
// symbol, void return, launch errors reported on stderr followed by exit(1)
// as the emitted CUDA_CHECK does, decode_attention_kivi_paged_library_flash.cu:9-12,
// :171).  The jacq_kivi_* symbols validate their arguments and return a
// status code; jacq_kivi_last_error() holds the message.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "jacq_kivi.h"
#include "kivi_kernels.h"

namespace {

using jacq::KiviGeo;

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

// Reference geometries: source_patch.py:660-671 (NH/NKV/TP2 local, HD,
// OLD_BLOCKS, BLOCK_SIZE, RESIDUAL).
constexpr jacq_kivi_geometry kGlobal = {40, 8, 128, 32, 32, 128, 124, INT32_MAX};
constexpr jacq_kivi_geometry kTp2Local = {20, 4, 128, 32, 32, 128, 124, INT32_MAX};

int64_t max_seq_len(const jacq_kivi_geometry& x) {
  return ((int64_t)x.max_pages_per_seq * x.page_size / jacq::kGroup) * jacq::kGroup + x.residual;
}

int check_geometry(const jacq_kivi_geometry* x) {
  if (!x) return fail(JACQ_KIVI_EINVAL, "geometry pointer is null");
  if (x->num_heads < 1 || x->num_kv_heads < 1 || x->num_heads % x->num_kv_heads != 0)
    return fail(JACQ_KIVI_EINVAL, "num_heads must be a positive multiple of num_kv_heads, got " +
                                      std::to_string(x->num_heads) + "/" +
                                      std::to_string(x->num_kv_heads));
  if (x->num_heads / x->num_kv_heads > 16)
    return fail(JACQ_KIVI_EINVAL, "query heads per kv head must be <= 16");
  if (x->head_dim != 64 && x->head_dim != 128)
    return fail(JACQ_KIVI_EINVAL, "head_dim must be 64 or 128, got " + std::to_string(x->head_dim));
  if (x->group_size != jacq::kGroup)
    return fail(JACQ_KIVI_EINVAL, "group_size must be 32 (int4 KIVI lane), got " +
                                      std::to_string(x->group_size));
  if (x->page_size != 16 && x->page_size != 32)
    return fail(JACQ_KIVI_EINVAL, "page_size must be 16 or 32 (a divisor of the 32-token group), got " +
                                      std::to_string(x->page_size));
  if (x->residual <= 0 || x->residual % x->group_size != 0)
    return fail(JACQ_KIVI_EINVAL, "residual must be a positive multiple of the group, got " +
                                      std::to_string(x->residual));
  if (x->max_pages_per_seq < 0) return fail(JACQ_KIVI_EINVAL, "max_pages_per_seq must be >= 0");
  if (x->num_pages < 1)
    return fail(JACQ_KIVI_EINVAL, "num_pages (page storage capacity) must be positive");
  if (jacq::split_count(max_seq_len(*x)) > 64)
    return fail(JACQ_KIVI_EINVAL, "block table addresses more than 64 x 4096 tokens per sequence");
  return JACQ_KIVI_OK;
}

KiviGeo make_geo(const jacq_kivi_geometry& x) {
  KiviGeo g;
  g.nh = x.num_heads;
  g.nkv = x.num_kv_heads;
  g.hd = x.head_dim;
  g.page = x.page_size;
  g.residual = x.residual;
  g.max_pages = x.max_pages_per_seq;
  g.num_pages = x.num_pages;
  g.gqa = x.num_heads / x.num_kv_heads;
  g.rs = x.residual + jacq::kGroup;
  g.lq = (int)(((int64_t)x.max_pages_per_seq * x.page_size / jacq::kGroup) * jacq::kGroup);
  return g;
}

// ---- per-device state: CU count, merge status word, library workspaces ----

// A library-owned split-K workspace, one per (device, stream): decodes on
// different streams may run at the same time and must not share partial
// slots.  An outgrown buffer is never freed (a captured graph may still hold
// its address); it moves to `retired` and lives until the process ends.
struct StreamWorkspace {
  hipStream_t stream;
  void* ptr;
  size_t bytes;
};
// Split-K workspace of jacq_kivi_decode_noalloc: a static device array, so
// that entry point allocates nothing.  Each device holds its own copy (at its
// own address, from hipGetSymbolAddress at set-up) until the process ends.
// Zero-initialised; like any workspace it needs no particular contents.
constexpr size_t kNoAllocScratchBytes = 32u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Split-K workspaces of the v1 decode symbols (jac_launch*), which allocate
// nothing either (the reference's launch contract: every buffer is the
// caller's, source_patch.py:2391-2417).  A static device array of
// kV1Regions regions; a stream takes the next free region on its first v1
// decode and keeps it (decodes on different streams may run at once, and a
// graph captured on a stream keeps its region's address).  A call whose
// queries need more than one region holds is split into launches of as many
// queries as fit, one after another on the stream (each query's result does
// not depend on which launch decodes it).
constexpr int kV1Regions = 8;
constexpr size_t kV1RegionBytes = 16u << 20;
static __device__ __align__(256) uint8_t v1_workspace[kV1Regions * kV1RegionBytes];

struct DeviceState {
  int cus = 0;
  void* scratch_ptr = nullptr;  // this device's copy of `scratch`
  // Pinned, host-coherent word the decode kernels set (system-scope vector
  // store) when a split-K merge wait runs out; read by the host without a
  // synchronisation, cleared by jacq_kivi_decode_status.
  volatile uint32_t* status = nullptr;
  uint32_t* status_dev = nullptr;  // the same word, as the device addresses it
  void* v1_ptr = nullptr;  // this device's copy of `v1_workspace`
  std::vector<hipStream_t> v1_streams;  // stream holding region i
  std::vector<StreamWorkspace> ws;
  std::vector<StreamWorkspace> retired;
};
std::mutex g_mu;
std::vector<DeviceState> g_dev;
// device allocations the library has made (jacq_kivi_test_device_allocations)
std::atomic<int64_t> g_device_allocations{0};

// Per-device set-up, once, with the device current.  Called by every entry
// point (and by jacq_kivi_init); everything it allocates lives until exit.
int init_device_locked(int dev) {
  if ((int)g_dev.size() <= dev) g_dev.resize(dev + 1);
  DeviceState& s = g_dev[dev];
  if (s.cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    s.cus = cus;
  }
  if (!s.status) {
    void* p = nullptr;
    if (hipHostMalloc(&p, 64, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess || !p)
      return fail(JACQ_KIVI_ENOMEM, "hipHostMalloc of the decode status word failed");
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess || !d)
      return fail(JACQ_KIVI_EHIP, "hipHostGetDevicePointer(status word) failed");
    *(volatile uint32_t*)p = 0;
    s.status = (volatile uint32_t*)p;
    s.status_dev = (uint32_t*)d;
  }
  if (!s.scratch_ptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr)
      return fail(JACQ_KIVI_EHIP, "hipGetSymbolAddress(scratch) failed");
    s.scratch_ptr = ptr;
  }
  if (!s.v1_ptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(v1_workspace)) != hipSuccess || !ptr)
      return fail(JACQ_KIVI_EHIP, "hipGetSymbolAddress(v1_workspace) failed");
    s.v1_ptr = ptr;
  }
  return JACQ_KIVI_OK;
}

// The v1 workspace region of `stream` on device `dev` (set up).
int v1_region(int dev, hipStream_t stream, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& s = g_dev[dev];
  size_t i = 0;
  while (i < s.v1_streams.size() && s.v1_streams[i] != stream) ++i;
  if (i == s.v1_streams.size()) {
    if (i == (size_t)kV1Regions)
      return fail(JACQ_KIVI_ENOMEM, "v1 decodes on more than " + std::to_string(kV1Regions) +
                                         " streams of one device (each stream keeps one of the "
                                         "library's static split-K workspace regions)");
    s.v1_streams.push_back(stream);
  }
  *out = (uint8_t*)s.v1_ptr + i * kV1RegionBytes;
  return JACQ_KIVI_OK;
}

int current_device(int* dev) {
  if (hipGetDevice(dev) != hipSuccess) return fail(JACQ_KIVI_EHIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_mu);
  return init_device_locked(*dev);
}

// Fields of a device set up by current_device (the vector may grow under
// other threads, so every read takes the lock).
struct DeviceInfo {
  int cus;
  volatile uint32_t* status;
  uint32_t* status_dev;
  void* scratch_ptr;
};
DeviceInfo device_state(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  const DeviceState& s = g_dev[dev];
  return {s.cus, s.status, s.status_dev, s.scratch_ptr};
}

// Set-up state of the current device without setting it up (nothing is
// allocated): false when jacq_kivi_init (or any other entry point) has not
// run on it yet.
bool device_ready(int* dev, DeviceInfo* info) {
  if (hipGetDevice(dev) != hipSuccess) return false;
  std::lock_guard<std::mutex> lk(g_mu);
  if ((int)g_dev.size() <= *dev) return false;
  const DeviceState& s = g_dev[*dev];
  if (!s.status || !s.scratch_ptr) return false;
  *info = {s.cus, s.status, s.status_dev, s.scratch_ptr};
  return true;
}

constexpr const char* kTimeoutMsg =
    "a split-K merge of an earlier decode on this device timed out and wrote NaN "
    "(its stream wavefronts never ran); call jacq_kivi_decode_status() to reset";

// Sequences the library's own split-K workspace covers from its first use
// (about 13 MB at the v1 geometry).
constexpr int kLibraryWorkspaceBatch = 256;
// Streams per device that may hold a library workspace at once.
constexpr int kLibraryWorkspaceStreams = 16;

int library_workspace(int dev, hipStream_t stream, size_t bytes, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  DeviceState& s = g_dev[dev];
  StreamWorkspace* w = nullptr;
  for (auto& x : s.ws)
    if (x.stream == stream) w = &x;
  if (!w) {
    if (s.ws.size() >= (size_t)kLibraryWorkspaceStreams)
      return fail(JACQ_KIVI_ENOMEM,
                  "library split-K workspaces exist for " + std::to_string(s.ws.size()) +
                      " streams of this device, the maximum; pass a workspace or call "
                      "jacq_kivi_release_workspaces()");
    s.ws.push_back({stream, nullptr, 0});
    w = &s.ws.back();
  }
  if (w->bytes < bytes) {
    if (w->ptr) s.retired.push_back(*w);
    w->ptr = nullptr;
    w->bytes = 0;
    const size_t want = bytes + bytes / 4;
    void* p = nullptr;
    // The first decode on a stream may be inside a stream capture (a graph
    // captured on a fresh stream); an allocation is not a stream operation,
    // so this thread's capture mode is relaxed around it, as the runtime
    // allows, instead of invalidating the capture.
    g_device_allocations.fetch_add(1, std::memory_order_relaxed);
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    const hipError_t me = hipMalloc(&p, want);
    if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (me != hipSuccess)
      return fail(JACQ_KIVI_ENOMEM, "hipMalloc of " + std::to_string(want) +
                                         " workspace bytes failed");
    // Not cleared: a flag counts only when it equals the launch's epoch (a
    // random 64-bit value with the top bit set), and a synchronous memset
    // could not run inside a stream capture, where this allocation may happen.
    w->ptr = p;
    w->bytes = want;
  }
  *out = w->ptr;
  return JACQ_KIVI_OK;
}

// Split slots per (sequence, kv head): split_plan never makes more than
// split_count(n) splits, which grows with n, so the longest sequence the call
// can see bounds every sequence's count.
struct SplitPlan {
  int max_splits;
  int runs_cap;  // per-query split: runs of the longest sequence (0: whole-call split)
};

SplitPlan plan_splits(int64_t max_tokens) { return {jacq::split_count(max_tokens), 0}; }

// Per-query split plan: a query of up to max_tokens tokens is cut into at
// most this many runs (the kernel's stream_waves of its units).
// A query of at most max_tokens tokens has T <= ceil(max_tokens / 32) tiles,
// at most R / 32 + 1 of them fp16 residual tiles, so its units (quantised
// groups + 3 per residual tile = T + 2 residual tiles) are bounded by
// T + 2 (R / 32 + 1) per kv head, whatever its length.
SplitPlan plan_splits_per_query(const KiviGeo& g, int64_t max_tokens, int waves) {
  const int64_t tiles = std::max<int64_t>(1, (max_tokens + jacq::kGroup - 1) / jacq::kGroup);
  const int64_t units = (int64_t)g.nkv * (tiles + 2 * (g.residual / jacq::kGroup + 1));
  const int64_t runs = std::min<int64_t>(waves, std::max<int64_t>(1, (units + 3) / 4));
  return {jacq::split_count(max_tokens), (int)runs};
}

// JACQ_KIVI_DECODE=simple selects the VALU decode kernel (a cross-check of
// the matrix-core kernel); the default is the matrix-core kernel.
bool use_simple_decode() {
  static const bool simple = [] {
    const char* e = std::getenv("JACQ_KIVI_DECODE");
    return e && std::string(e) == "simple";
  }();
  return simple;
}

// Partial-result slots: VALU kernel -- one per (sequence, kv head, split);
// matrix-core kernel -- one per (sequence, kv head) plus one per wavefront
// (a wavefront's run cuts at most one extra piece off the stream).
// Per-query split (the v1 symbols): one per (query, kv head) plus one per
// run of each query, at most runs_cap (the runs of the longest sequence).
size_t partial_slots(const KiviGeo& g, int batch, const SplitPlan& sp, int waves) {
  if (use_simple_decode())
    return sp.max_splits <= 1 ? 0 : (size_t)batch * g.nkv * sp.max_splits;
  if (sp.runs_cap > 0) return (size_t)batch * ((size_t)g.nkv + (size_t)sp.runs_cap);
  return (size_t)batch * g.nkv + (size_t)waves;
}

// Workspace: [m,l fp32 per slot and head][acc fp32 per slot, head, channel]
// and, for the matrix-core kernel, [epoch uint64 per slot] (8-byte aligned:
// G * (HD + 2) floats per slot is even).  The flags need no initial contents:
// a flag counts only when it holds the current launch's 64-bit epoch.
// A 16-byte header comes first: the poison word the matrix-core kernel's
// merge sets when a wait runs out (it must sit at the same place whatever the
// batch of the calls sharing the workspace).
constexpr size_t kWorkspaceHeader = 16;

size_t workspace_bytes(const KiviGeo& g, int batch, const SplitPlan& sp, int waves) {
  const size_t slots = partial_slots(g, batch, sp, waves);
  if (slots == 0) return 0;
  const size_t flags = use_simple_decode() ? 0 : slots * sizeof(uint64_t);
  return kWorkspaceHeader + slots * g.gqa * (size_t)(g.hd + 2) * sizeof(float) + flags;
}

void fill_ws(jacq::DecodeArgs& a, const KiviGeo& g, int batch, const SplitPlan& sp, int waves,
             void* ws) {
  a.max_splits = sp.max_splits;
  a.batch = batch;
  a.waves = waves;
  a.per_query = sp.runs_cap > 0;
  const size_t slots = partial_slots(g, batch, sp, waves) * g.gqa;
  a.ws_poison = (uint64_t*)ws;
  a.ws_ml = ws ? (float*)((uint8_t*)ws + kWorkspaceHeader) : nullptr;
  a.ws_acc = ws ? a.ws_ml + slots * 2 : nullptr;
  a.ws_flag = ws ? (uint64_t*)(a.ws_acc + slots * g.hd) : nullptr;
}

// Fused write + decode: the first stream wavefronts do the writer's work
// before their (shorter) runs (about one per 8 (sequence, kv head, K | V)
// pairs, at most 128), and one epoch flag per
// age-out item (sequence, kv head, K | V, 32-channel slice) after the split-K
// workspace.
int step_writer_waves(const KiviGeo& g, int batch) {
  return std::max(1, std::min(128, 2 * batch * g.nkv / 8));
}
size_t step_flag_bytes(const KiviGeo& g, int batch) {
  // K and V, one per 32-channel slice each
  return (size_t)2 * (g.hd / jacq::kGroup) * batch * g.nkv * sizeof(uint64_t);
}

// ---- measurement hook: HIP events around the decode ----
// While enabled, each decode call takes the next triple of a pre-created
// event pool and uses it on the call's own stream: before the decode, a
// middle event in split mode only, and after the decode.  In split mode the
// matrix-core decode (one kernel) is launched with the first two as the
// start / stop events the command processor stamps at the kernel's own start
// and end; the VALU decode records the middle one between its kernel and its
// merge.  Split mode delays the next kernel by a few microseconds.
struct Profiler {
  bool on = false;
  bool split = true;
  int used = 0, wused = 0;
  std::vector<hipEvent_t> ev;   // decode: 3 per call
  std::vector<hipEvent_t> wev;  // cache write: 2 per call
};
std::mutex g_prof_mu;
Profiler g_prof;

void profile_slot(hipEvent_t out[3]) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (!g_prof.on || 3 * (g_prof.used + 1) > (int)g_prof.ev.size()) return;
  for (int i = 0; i < 3; ++i) out[i] = g_prof.ev[3 * g_prof.used + i];
  if (!g_prof.split) out[1] = nullptr;
  ++g_prof.used;
}

void profile_write_slot(hipEvent_t out[2]) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  if (!g_prof.on || 2 * (g_prof.wused + 1) > (int)g_prof.wev.size()) return;
  for (int i = 0; i < 2; ++i) out[i] = g_prof.wev[2 * g_prof.wused + i];
  ++g_prof.wused;
}

// The kernels move Q, O, codes, scales, scratch and new tokens in 16-byte
// vectors (and the workspace in float4), so every base address must be
// 16-byte aligned; torch allocations and their row slices are.
static bool aligned16(std::initializer_list<const void*> ps) {
  uintptr_t bits = 0;
  for (const void* p : ps) bits |= (uintptr_t)p;
  return (bits & 15u) == 0;
}

// Decode with a runtime geometry; seq_len_host >= 0 when the (single) length
// is known on the host, which tightens the split plan.  retained_pages >= 0
// selects the sparse-retained window (bt is then the compact table).
int run_decode(const jacq_kivi_geometry& x, const jacq_half_t* Q, const int32_t* seq_lens,
               int seq_len_host, const int32_t* bt, int64_t bt_stride, const uint8_t* kc,
               const jacq_half_t* ksc, const jacq_half_t* kz, const uint8_t* vc,
               const jacq_half_t* vsc, const jacq_half_t* vz, const jacq_half_t* kscr,
               const jacq_half_t* vscr, int64_t scr_stride, int batch, float* O, void* ws,
               size_t ws_bytes, hipStream_t stream, int retained_pages = -1,
               bool per_query = false, const jacq::AppendArgs* step = nullptr) {
  if (!aligned16({Q, O, kc, ksc, kz, vc, vsc, vz, kscr, vscr, ws}))
    return fail(JACQ_KIVI_EINVAL, "tensor and workspace pointers must be 16-byte aligned");
  const KiviGeo g = make_geo(x);
  int dev = 0;
  if (int e = current_device(&dev)) return e;
  const DeviceInfo ds = device_state(dev);
  if (*ds.status != 0) return fail(JACQ_KIVI_ETIMEOUT, kTimeoutMsg);
  int64_t max_tokens = max_seq_len(x);
  if (seq_len_host >= 0) {
    int ov, rv;
    jacq::window_of(g, retained_pages, seq_len_host, &ov, &rv);
    max_tokens = ov + rv;
  }
  const int waves = jacq::decode_stream_waves(g, ds.cus);  // writer wavefronts included
  // the writer wavefronts are stream wavefronts: never more than the grid holds
  const int nw = step ? std::min(step_writer_waves(g, batch), waves) : 0;
  const SplitPlan sp =
      per_query ? plan_splits_per_query(g, max_tokens, waves) : plan_splits(max_tokens);
  const size_t need = workspace_bytes(g, batch, sp, waves) + (step ? step_flag_bytes(g, batch) : 0);
  if (need > 0) {
    if (ws == nullptr) {
      // sized for at least kLibraryWorkspaceBatch sequences on first use, so
      // that later calls up to that batch (graph captures included) do not
      // allocate
      const size_t want =
          std::max(need, workspace_bytes(g, std::max(batch, kLibraryWorkspaceBatch), sp, waves));
      if (int e = library_workspace(dev, stream, want, &ws)) return e;
    } else if (ws_bytes < need) {
      return fail(JACQ_KIVI_ENOMEM, "workspace of " + std::to_string(ws_bytes) +
                                         " bytes is smaller than the " + std::to_string(need) +
                                         " required");
    }
  }
  jacq::DecodeArgs a{};
  a.q = Q;
  a.q_stride = (int64_t)g.nh * g.hd;
  a.seq_lens = seq_lens;
  a.seq_len = seq_len_host;
  a.block_tables = bt;
  a.bt_stride = bt_stride;
  a.k_code = kc;
  a.k_scale = ksc;
  a.k_zero = kz;
  a.v_code = vc;
  a.v_scale = vsc;
  a.v_zero = vz;
  a.k_scr = kscr;
  a.v_scr = vscr;
  a.scr_stride = scr_stride;
  a.out = O;
  a.out_stride = (int64_t)g.nh * g.hd;
  a.retained_pages = retained_pages;
  a.status = ds.status_dev;
  fill_ws(a, g, batch, sp, waves, need > 0 ? ws : nullptr);
  if (step) {
    a.wr = *step;
    a.writer_waves = nw;
    // the writer flags follow the split-K workspace
    a.ws_wflag = (uint64_t*)((uint8_t*)ws + (need - step_flag_bytes(g, batch)));
  }
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
  profile_slot(ev);
  hipError_t e;
  if (use_simple_decode()) {
    if (ev[0] && hipEventRecord(ev[0], stream) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "hipEventRecord failed");
    e = jacq::launch_decode(g, a, batch, stream, ev[1]);
    if (e == hipSuccess && ev[2] && hipEventRecord(ev[2], stream) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "hipEventRecord failed");
  } else {
    e = jacq::launch_decode_mfma(g, a, batch, stream, {ev[0], ev[1], ev[2]});
  }
  if (e != hipSuccess) return fail(JACQ_KIVI_EHIP, "decode launch failed");
  return JACQ_KIVI_OK;
}

int run_append(const jacq_kivi_geometry& x, uint8_t* kc, jacq_half_t* ksc, jacq_half_t* kz,
               uint8_t* vc, jacq_half_t* vsc, jacq_half_t* vz, jacq_half_t* kscr,
               jacq_half_t* vscr, int64_t scr_stride, const jacq_half_t* nk,
               const jacq_half_t* nv, int64_t new_stride, const int32_t* bt, int64_t bt_stride,
               const int32_t* start_lens, int start_len, int num_new, int batch,
               hipStream_t stream) {
  if (!aligned16({kc, ksc, kz, vc, vsc, vz, kscr, vscr, nk, nv}))
    return fail(JACQ_KIVI_EINVAL, "tensor pointers must be 16-byte aligned");
  const KiviGeo g = make_geo(x);
  jacq::AppendArgs a{};
  a.k_code = kc;
  a.k_scale = ksc;
  a.k_zero = kz;
  a.v_code = vc;
  a.v_scale = vsc;
  a.v_zero = vz;
  a.k_scr = kscr;
  a.v_scr = vscr;
  a.scr_stride = scr_stride;
  a.new_k = nk;
  a.new_v = nv;
  a.new_stride = new_stride;
  a.block_tables = bt;
  a.bt_stride = bt_stride;
  a.start_lens = start_lens;
  a.start_len = start_len;
  a.num_new = num_new;
  hipEvent_t ev[2] = {nullptr, nullptr};
  profile_write_slot(ev);
  if (ev[0] && hipEventRecord(ev[0], stream) != hipSuccess)
    return fail(JACQ_KIVI_EHIP, "hipEventRecord failed");
  if (jacq::launch_append(g, a, batch, stream) != hipSuccess)
    return fail(JACQ_KIVI_EHIP, "cache-write launch failed");
  if (ev[1] && hipEventRecord(ev[1], stream) != hipSuccess)
    return fail(JACQ_KIVI_EHIP, "hipEventRecord failed");
  return JACQ_KIVI_OK;
}

// Decode of the v1 symbols: the per-query split (every query decodes to the
// same bits whatever else the call holds) and the stream's static workspace
// region, so nothing is allocated.  Queries beyond what one region holds go
// to further launches on the stream.
int v1_decode(const jacq_kivi_geometry& x, const jacq_half_t* Q, const int32_t* seq_lens,
              int seq_len_host, const int32_t* bt, const uint8_t* kc, const jacq_half_t* ksc,
              const jacq_half_t* kz, const uint8_t* vc, const jacq_half_t* vsc,
              const jacq_half_t* vz, const jacq_half_t* kscr, const jacq_half_t* vscr,
              int queries, float* O, hipStream_t stream, int retained_pages = -1) {
  int dev = 0;
  if (int e = current_device(&dev)) return e;
  void* region = nullptr;
  if (int e = v1_region(dev, stream, &region)) return e;
  const KiviGeo g = make_geo(x);
  const int waves = jacq::decode_stream_waves(g, device_state(dev).cus);
  const SplitPlan sp = plan_splits_per_query(g, max_seq_len(x), waves);
  const size_t one = workspace_bytes(g, 1, sp, waves);
  const size_t per = one > kWorkspaceHeader ? one - kWorkspaceHeader : 0;
  const int chunk =
      per == 0 ? queries
               : (int)std::min<size_t>((size_t)queries, (kV1RegionBytes - kWorkspaceHeader) / per);
  if (chunk < 1) return fail(JACQ_KIVI_ENOMEM, "one query needs more than a v1 workspace region");
  const int64_t qs = (int64_t)g.nh * g.hd;
  for (int q0 = 0; q0 < queries; q0 += chunk) {
    const int n = std::min(chunk, queries - q0);
    if (int e = run_decode(x, Q + q0 * qs, seq_lens ? seq_lens + q0 : nullptr, seq_len_host, bt, 0,
                           kc, ksc, kz, vc, vsc, vz, kscr, vscr, 0, n, O + q0 * qs, region,
                           kV1RegionBytes, stream, retained_pages, true))
      return e;
  }
  return JACQ_KIVI_OK;
}

// CUDA_CHECK of the emitted v1 symbols: report and exit(1).  A merge
// time-out of an earlier decode is reported the same way by the next v1
// decode on the device.
void v1_check(int status, const char* where) {
  if (status == JACQ_KIVI_OK) return;
  if (status == JACQ_KIVI_EHIP) {
    const hipError_t e = hipGetLastError();
    std::fprintf(stderr, "HIP error %s in %s: %s\n", hipGetErrorString(e), where,
                 g_last_error.c_str());
  } else {
    std::fprintf(stderr, "jacq_kivi error %d in %s: %s\n", status, where, g_last_error.c_str());
  }
  std::exit(1);
}

}  // namespace

extern "C" {

int jacq_kivi_abi_version(void) { return JACQ_KIVI_ABI_VERSION; }
int jacq_kivi_ext_version(void) { return JACQ_KIVI_EXT_VERSION; }
const char* jacq_kivi_last_error(void) { return g_last_error.c_str(); }

int jacq_kivi_check_geometry(const jacq_kivi_geometry* geo) { return check_geometry(geo); }

int jacq_kivi_init(void) {
  int dev = 0;
  return current_device(&dev);
}

int jacq_kivi_decode_status(void* workspace, size_t workspace_bytes_, hipStream_t stream) {
  int dev = 0;
  if (int e = current_device(&dev)) return e;
  if (hipStreamSynchronize(stream) != hipSuccess)
    return fail(JACQ_KIVI_EHIP, "hipStreamSynchronize failed");
  const DeviceInfo ds = device_state(dev);
  if (*ds.status == 0) return JACQ_KIVI_OK;
  // Reset: a timed-out merge left flags that its stream wavefronts set after
  // it gave up; a graph replay (same epoch) would take them for its own.
  // Every workspace the device's decodes may have used is cleared.
  if (hipDeviceSynchronize() != hipSuccess) return fail(JACQ_KIVI_EHIP, "hipDeviceSynchronize failed");
  std::vector<StreamWorkspace> all;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    all = g_dev[dev].ws;
    all.insert(all.end(), g_dev[dev].retired.begin(), g_dev[dev].retired.end());
    all.push_back({stream, g_dev[dev].scratch_ptr, kNoAllocScratchBytes});
    all.push_back({stream, g_dev[dev].v1_ptr, kV1Regions * kV1RegionBytes});
  }
  if (workspace && workspace_bytes_) all.push_back({stream, workspace, workspace_bytes_});
  for (const auto& w : all)
    if (w.ptr && hipMemset(w.ptr, 0, w.bytes) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "hipMemset(workspace) failed");
  *ds.status = 0;
  return fail(JACQ_KIVI_ETIMEOUT, "a split-K merge timed out since the last query; its "
                                  "outputs were NaN; the workspaces are reset");
}

int jacq_kivi_release_workspaces(void) {
  int dev = 0;
  if (int e = current_device(&dev)) return e;
  if (hipDeviceSynchronize() != hipSuccess) return fail(JACQ_KIVI_EHIP, "hipDeviceSynchronize failed");
  std::vector<StreamWorkspace> all;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    all.swap(g_dev[dev].ws);
    all.insert(all.end(), g_dev[dev].retired.begin(), g_dev[dev].retired.end());
    g_dev[dev].retired.clear();
  }
  for (const auto& w : all)
    if (w.ptr && hipFree(w.ptr) != hipSuccess) return fail(JACQ_KIVI_EHIP, "hipFree failed");
  return JACQ_KIVI_OK;
}

int64_t jacq_kivi_test_device_allocations(void) {
  return g_device_allocations.load(std::memory_order_relaxed);
}

void jacq_kivi_test_force_merge_timeout(uint32_t microseconds) {
  jacq::set_test_merge_timeout_us(microseconds);
}

int64_t jacq_kivi_max_seq_len(const jacq_kivi_geometry* geo) {
  if (check_geometry(geo) != JACQ_KIVI_OK) return -1;
  return max_seq_len(*geo);
}

int jacq_kivi_check_block_table_width(const jacq_kivi_geometry* geo, int64_t width,
                                      int64_t seq_len) {
  if (int e = check_geometry(geo)) return e;
  const int64_t cap = max_seq_len(*geo);
  if (seq_len < 1 || seq_len > cap)
    return fail(JACQ_KIVI_EINVAL, "SEQ_LEN must be in [1, " + std::to_string(cap) +
                                      "] for KIVI BLOCK_TABLE validation");
  const int64_t required =
      seq_len > geo->residual
          ? ((seq_len - geo->residual) / geo->group_size) * geo->group_size / geo->page_size
          : 0;
  if (width < required)
    return fail(JACQ_KIVI_EINVAL, "BLOCK_TABLE dim 0 must be at least " + std::to_string(required) +
                                      ", got " + std::to_string(width));
  return JACQ_KIVI_OK;
}

size_t jacq_kivi_decode_workspace_size(const jacq_kivi_geometry* geo, int32_t batch) {
  if (check_geometry(geo) != JACQ_KIVI_OK || batch < 1) return 0;
  int dev = 0;
  if (current_device(&dev) != JACQ_KIVI_OK) return 0;
  const KiviGeo g = make_geo(*geo);
  return workspace_bytes(g, batch, plan_splits(max_seq_len(*geo)),
                         jacq::decode_stream_waves(g, device_state(dev).cus));
}

int jacq_kivi_profile_wave_stamps(uint64_t* buffer, int32_t capacity) {
  if (buffer && capacity < 1) return fail(JACQ_KIVI_EINVAL, "capacity must be >= 1");
  jacq::set_wave_stamps(buffer, buffer ? capacity : 0);
  return JACQ_KIVI_OK;
}

int jacq_kivi_decode(const jacq_kivi_geometry* geo, const jacq_half_t* Q, const int32_t* SEQ_LENS,
                     const int32_t* BLOCK_TABLES, const uint8_t* K_CODE_PAGES,
                     const jacq_half_t* K_SCALE_PAGES, const jacq_half_t* K_ZERO_PAGES,
                     const uint8_t* V_CODE_PAGES, const jacq_half_t* V_SCALE_PAGES,
                     const jacq_half_t* V_ZERO_PAGES, const jacq_half_t* K_RESIDUAL_SCRATCH,
                     const jacq_half_t* V_RESIDUAL_SCRATCH, int32_t batch, float* O,
                     void* workspace, size_t workspace_bytes_, hipStream_t stream) {
  if (int e = check_geometry(geo)) return e;
  if (batch < 1) return fail(JACQ_KIVI_EINVAL, "batch must be >= 1");
  if (!Q || !SEQ_LENS || !K_CODE_PAGES || !K_SCALE_PAGES || !K_ZERO_PAGES || !V_CODE_PAGES ||
      !V_SCALE_PAGES || !V_ZERO_PAGES || !K_RESIDUAL_SCRATCH || !V_RESIDUAL_SCRATCH || !O ||
      (!BLOCK_TABLES && geo->max_pages_per_seq > 0))
    return fail(JACQ_KIVI_EINVAL, "null tensor pointer");
  const int64_t scr = (int64_t)geo->num_kv_heads * (geo->residual + geo->group_size) * geo->head_dim;
  return run_decode(*geo, Q, SEQ_LENS, -1, BLOCK_TABLES, geo->max_pages_per_seq, K_CODE_PAGES,
                    K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES,
                    K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, scr, batch, O, workspace,
                    workspace_bytes_, stream);
}

size_t jacq_kivi_write_decode_workspace_size(const jacq_kivi_geometry* geo, int32_t batch) {
  if (check_geometry(geo) != JACQ_KIVI_OK || batch < 1) return 0;
  int dev = 0;
  if (current_device(&dev) != JACQ_KIVI_OK) return 0;
  const KiviGeo g = make_geo(*geo);
  const int waves = jacq::decode_stream_waves(g, device_state(dev).cus);
  return workspace_bytes(g, batch, plan_splits(max_seq_len(*geo)), waves) +
         step_flag_bytes(g, batch);
}

int jacq_kivi_write_decode(const jacq_kivi_geometry* geo, const jacq_half_t* Q,
                           const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                           const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLES,
                           uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                           jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                           jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                           jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                           int32_t batch, float* O, void* workspace, size_t workspace_bytes_,
                           hipStream_t stream) {
  if (int e = check_geometry(geo)) return e;
  if (batch < 1) return fail(JACQ_KIVI_EINVAL, "batch must be >= 1");
  if (!Q || !NEW_K || !NEW_V || !SEQ_LENS || !K_CODE_PAGES || !K_SCALE_PAGES || !K_ZERO_PAGES ||
      !V_CODE_PAGES || !V_SCALE_PAGES || !V_ZERO_PAGES || !K_RESIDUAL_SCRATCH ||
      !V_RESIDUAL_SCRATCH || !O || (!BLOCK_TABLES && geo->max_pages_per_seq > 0))
    return fail(JACQ_KIVI_EINVAL, "null tensor pointer");
  if (!aligned16({NEW_K, NEW_V}))
    return fail(JACQ_KIVI_EINVAL, "tensor pointers must be 16-byte aligned");
  const int64_t scr = (int64_t)geo->num_kv_heads * (geo->residual + geo->group_size) * geo->head_dim;
  jacq::AppendArgs w{};
  w.k_code = K_CODE_PAGES;
  w.k_scale = K_SCALE_PAGES;
  w.k_zero = K_ZERO_PAGES;
  w.v_code = V_CODE_PAGES;
  w.v_scale = V_SCALE_PAGES;
  w.v_zero = V_ZERO_PAGES;
  w.k_scr = K_RESIDUAL_SCRATCH;
  w.v_scr = V_RESIDUAL_SCRATCH;
  w.scr_stride = scr;
  w.new_k = NEW_K;
  w.new_v = NEW_V;
  w.new_stride = (int64_t)geo->num_kv_heads * geo->head_dim;
  w.block_tables = BLOCK_TABLES;
  w.bt_stride = geo->max_pages_per_seq;
  w.start_lens = nullptr;  // SEQ_LENS - 1, read by the kernel
  w.num_new = 1;
  if (use_simple_decode())
    return fail(JACQ_KIVI_EINVAL, "the fused write + decode runs on the matrix-core decode only");
  return run_decode(*geo, Q, SEQ_LENS, -1, BLOCK_TABLES, geo->max_pages_per_seq, K_CODE_PAGES,
                    K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES,
                    K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, scr, batch, O, workspace,
                    workspace_bytes_, stream, -1, false, &w);
}

int jacq_kivi_decode_noalloc(const jacq_kivi_geometry* geo, const jacq_half_t* Q,
                             const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLES,
                             const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                             const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                             const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                             const jacq_half_t* K_RESIDUAL_SCRATCH,
                             const jacq_half_t* V_RESIDUAL_SCRATCH, int32_t batch, float* O,
                             hipStream_t stream) {
  if (int e = check_geometry(geo)) return e;
  if (batch < 1) return fail(JACQ_KIVI_EINVAL, "batch must be >= 1");
  int dev = 0;
  DeviceInfo ds{};
  if (!device_ready(&dev, &ds))
    return fail(JACQ_KIVI_EINVAL,
                "jacq_kivi_decode_noalloc: call jacq_kivi_init() on this device first "
                "(its one-time set-up is the only allocation)");
  const KiviGeo g = make_geo(*geo);
  const size_t need = workspace_bytes(g, batch, plan_splits(max_seq_len(*geo)),
                                      jacq::decode_stream_waves(g, ds.cus));
  if (need > kNoAllocScratchBytes)
    return fail(JACQ_KIVI_ENOMEM,
                "jacq_kivi_decode_noalloc: " + std::to_string(batch) +
                    " sequences at this geometry need " + std::to_string(need) +
                    " bytes of split-K workspace, above the static " +
                    std::to_string(kNoAllocScratchBytes) +
                    "-byte maximum; use jacq_kivi_decode with a workspace");
  if (!Q || !SEQ_LENS || !K_CODE_PAGES || !K_SCALE_PAGES || !K_ZERO_PAGES || !V_CODE_PAGES ||
      !V_SCALE_PAGES || !V_ZERO_PAGES || !K_RESIDUAL_SCRATCH || !V_RESIDUAL_SCRATCH || !O ||
      (!BLOCK_TABLES && geo->max_pages_per_seq > 0))
    return fail(JACQ_KIVI_EINVAL, "null tensor pointer");
  const int64_t scr = (int64_t)geo->num_kv_heads * (geo->residual + geo->group_size) * geo->head_dim;
  return run_decode(*geo, Q, SEQ_LENS, -1, BLOCK_TABLES, geo->max_pages_per_seq, K_CODE_PAGES,
                    K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES,
                    K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, scr, batch, O, ds.scratch_ptr,
                    kNoAllocScratchBytes, stream);
}

int jacq_kivi_decode_sparse_retained(
    const jacq_kivi_geometry* geo, const jacq_half_t* Q, int32_t SEQ_LEN,
    const int32_t* RETAINED_BLOCK_TABLE, int32_t NUM_RETAINED_PAGES,
    const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
    const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
    const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
    const jacq_half_t* K_RESIDUAL_SCRATCH, const jacq_half_t* V_RESIDUAL_SCRATCH, float* O,
    void* workspace, size_t workspace_bytes_, hipStream_t stream) {
  if (int e = check_geometry(geo)) return e;
  if (NUM_RETAINED_PAGES < 0 || NUM_RETAINED_PAGES > geo->max_pages_per_seq)
    return fail(JACQ_KIVI_EINVAL, "NUM_RETAINED_PAGES must be in [0, max_pages_per_seq = " +
                                      std::to_string(geo->max_pages_per_seq) + "], got " +
                                      std::to_string(NUM_RETAINED_PAGES));
  if (NUM_RETAINED_PAGES > geo->num_pages)
    return fail(JACQ_KIVI_EINVAL,
                "NUM_RETAINED_PAGES cannot exceed physical page storage capacity");
  const int64_t cap = max_seq_len(*geo);
  if (SEQ_LEN < 1 || SEQ_LEN > cap)
    return fail(JACQ_KIVI_EINVAL, "SEQ_LEN must be in [1, " + std::to_string(cap) + "], got " +
                                      std::to_string(SEQ_LEN));
  if (!Q || !K_CODE_PAGES || !K_SCALE_PAGES || !K_ZERO_PAGES || !V_CODE_PAGES ||
      !V_SCALE_PAGES || !V_ZERO_PAGES || !K_RESIDUAL_SCRATCH || !V_RESIDUAL_SCRATCH || !O ||
      (!RETAINED_BLOCK_TABLE && NUM_RETAINED_PAGES > 0))
    return fail(JACQ_KIVI_EINVAL, "null tensor pointer");
  return run_decode(*geo, Q, nullptr, SEQ_LEN, RETAINED_BLOCK_TABLE, 0, K_CODE_PAGES,
                    K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES,
                    K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, 0, 1, O, workspace,
                    workspace_bytes_, stream, NUM_RETAINED_PAGES);
}

int jacq_kivi_cache_append(const jacq_kivi_geometry* geo, uint8_t* K_CODE_PAGES,
                           jacq_half_t* K_SCALE_PAGES, jacq_half_t* K_ZERO_PAGES,
                           uint8_t* V_CODE_PAGES, jacq_half_t* V_SCALE_PAGES,
                           jacq_half_t* V_ZERO_PAGES, jacq_half_t* K_RESIDUAL_SCRATCH,
                           jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                           const jacq_half_t* NEW_V, const int32_t* BLOCK_TABLES,
                           const int32_t* START_LENS, int32_t num_new, int32_t batch,
                           hipStream_t stream) {
  if (int e = check_geometry(geo)) return e;
  if (batch < 1) return fail(JACQ_KIVI_EINVAL, "batch must be >= 1");
  if (num_new < 1) return fail(JACQ_KIVI_EINVAL, "num_new must be >= 1");
  if (!K_CODE_PAGES || !K_SCALE_PAGES || !K_ZERO_PAGES || !V_CODE_PAGES || !V_SCALE_PAGES ||
      !V_ZERO_PAGES || !K_RESIDUAL_SCRATCH || !V_RESIDUAL_SCRATCH || !NEW_K || !NEW_V ||
      !START_LENS || (!BLOCK_TABLES && geo->max_pages_per_seq > 0))
    return fail(JACQ_KIVI_EINVAL, "null tensor pointer");
  const int64_t scr = (int64_t)geo->num_kv_heads * (geo->residual + geo->group_size) * geo->head_dim;
  const int64_t nst = (int64_t)num_new * geo->num_kv_heads * geo->head_dim;
  return run_append(*geo, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES,
                    V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, scr, NEW_K, NEW_V, nst,
                    BLOCK_TABLES, geo->max_pages_per_seq, START_LENS, 0, num_new, batch, stream);
}

int jacq_kivi_profile_start(int32_t max_calls, int32_t split) {
  if (max_calls < 1) return fail(JACQ_KIVI_EINVAL, "max_calls must be >= 1");
  std::lock_guard<std::mutex> lk(g_prof_mu);
  for (auto* pool : {&g_prof.ev, &g_prof.wev}) {
    const size_t want = (pool == &g_prof.ev ? 3u : 2u) * (size_t)max_calls;
    while (pool->size() < want) {
      hipEvent_t e = nullptr;
      if (hipEventCreate(&e) != hipSuccess) return fail(JACQ_KIVI_EHIP, "hipEventCreate failed");
      pool->push_back(e);
    }
  }
  g_prof.used = 0;
  g_prof.wused = 0;
  g_prof.split = split != 0;
  g_prof.on = true;
  return JACQ_KIVI_OK;
}

int32_t jacq_kivi_profile_stop(float* kernel_ms, float* merge_ms, int32_t cap) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  g_prof.on = false;
  const int n = g_prof.used < cap ? g_prof.used : cap;
  for (int i = 0; i < n; ++i) {
    hipEvent_t* e = &g_prof.ev[3 * i];
    if (hipEventSynchronize(e[2]) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "event timing failed");
    if (!g_prof.split) {  // the whole decode in kernel_ms
      merge_ms[i] = 0.0f;
      if (hipEventElapsedTime(&kernel_ms[i], e[0], e[2]) != hipSuccess)
        return fail(JACQ_KIVI_EHIP, "event timing failed");
      continue;
    }
    if (hipEventElapsedTime(&kernel_ms[i], e[0], e[1]) != hipSuccess ||
        hipEventElapsedTime(&merge_ms[i], e[1], e[2]) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "event timing failed");
  }
  g_prof.used = 0;
  return n;
}

int32_t jacq_kivi_profile_write_ms(float* ms, int32_t cap) {
  std::lock_guard<std::mutex> lk(g_prof_mu);
  const int n = g_prof.wused < cap ? g_prof.wused : cap;
  for (int i = 0; i < n; ++i) {
    hipEvent_t* e = &g_prof.wev[2 * i];
    if (hipEventSynchronize(e[1]) != hipSuccess ||
        hipEventElapsedTime(&ms[i], e[0], e[1]) != hipSuccess)
      return fail(JACQ_KIVI_EHIP, "event timing failed");
  }
  g_prof.wused = 0;
  return n;
}

// plan_batched_write, source_patch.py:504-553.
int32_t jacq_kivi_plan_batched_write(int32_t start_seq_len, int32_t num_new, int32_t residual,
                                     int32_t group, jacq_kivi_subchunk* out, int32_t cap) {
  if (start_seq_len < 0)
    return fail(-1, "start_seq_len must be >= 0, got " + std::to_string(start_seq_len));
  if (num_new < 1) return fail(-1, "num_new_tokens must be >= 1, got " + std::to_string(num_new));
  if (residual <= 0 || group <= 0) return fail(-1, "residual and block_size must be positive");
  auto split = [&](int32_t L) {
    const int32_t q = L - residual;
    return q < 0 ? 0 : (q / group) * group;
  };
  const int32_t capacity = residual + group;
  int32_t n = 0, seq_len = start_seq_len, remaining = num_new;
  while (remaining > 0) {
    const int32_t prev_old = split(seq_len);
    const int32_t prev_res = seq_len - prev_old;
    const int32_t room = capacity - prev_res;
    const int32_t take = remaining < room ? remaining : room;
    if (take <= 0)
      return fail(-1, "planning invariant violated: no room to append even one token "
                      "(prev_residual_len=" + std::to_string(prev_res) +
                      ", scratch_capacity=" + std::to_string(capacity) + ")");
    const int32_t new_len = seq_len + take;
    const int32_t next_old = split(new_len);
    if (n >= cap) return fail(-1, "sub-chunk buffer too small");
    out[n].start_seq_len = seq_len;
    out[n].num_new = take;
    out[n].scratch_start = prev_res;
    out[n].age_out_page = next_old > prev_old ? prev_old / group : -1;
    out[n].post_shift_residual_len = next_old > prev_old ? new_len - next_old : -1;
    ++n;
    seq_len = new_len;
    remaining -= take;
  }
  return n;
}

// ---- reference contract, ABI v1 ----

void jac_launch(const jacq_half_t* Q, const int32_t* BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
                const jacq_half_t* K_SCALE_PAGES, const jacq_half_t* K_ZERO_PAGES,
                const uint8_t* V_CODE_PAGES, const jacq_half_t* V_SCALE_PAGES,
                const jacq_half_t* V_ZERO_PAGES, const jacq_half_t* K_RESIDUAL_SCRATCH,
                const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN, float* O,
                hipStream_t stream) {
  v1_check(v1_decode(kGlobal, Q, nullptr, SEQ_LEN, BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES,
                     K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH,
                     V_RESIDUAL_SCRATCH, 1, O, stream),
           "jac_launch");
}

void jac_launch_tp2_local(const jacq_half_t* Q, const int32_t* BLOCK_TABLE,
                          const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                          const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                          const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                          const jacq_half_t* K_RESIDUAL_SCRATCH,
                          const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN, float* O,
                          hipStream_t stream) {
  v1_check(v1_decode(kTp2Local, Q, nullptr, SEQ_LEN, BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES,
                     K_ZERO_PAGES, V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH,
                     V_RESIDUAL_SCRATCH, 1, O, stream),
           "jac_launch_tp2_local");
}

static void sparse_v1(const jacq_kivi_geometry& x, const jacq_half_t* Q,
                      const int32_t* RETAINED_BLOCK_TABLE, const uint8_t* kc,
                      const jacq_half_t* ks, const jacq_half_t* kz, const uint8_t* vc,
                      const jacq_half_t* vs, const jacq_half_t* vz, const jacq_half_t* kscr,
                      const jacq_half_t* vscr, int SEQ_LEN, int NUM_RETAINED_PAGES, float* O,
                      hipStream_t stream, const char* where) {
  // the kernel clamps NUM_RETAINED_PAGES to [0, dense old pages] itself
  v1_check(v1_decode(x, Q, nullptr, SEQ_LEN, RETAINED_BLOCK_TABLE, kc, ks, kz, vc, vs, vz, kscr,
                     vscr, 1, O, stream, NUM_RETAINED_PAGES < 0 ? 0 : NUM_RETAINED_PAGES),
           where);
}

void jac_launch_sparse_retained(const jacq_half_t* Q, const int32_t* RETAINED_BLOCK_TABLE,
                                const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                                const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                                const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                                const jacq_half_t* K_RESIDUAL_SCRATCH,
                                const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN,
                                int NUM_RETAINED_PAGES, float* O, hipStream_t stream) {
  sparse_v1(kGlobal, Q, RETAINED_BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
            V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH,
            SEQ_LEN, NUM_RETAINED_PAGES, O, stream, "jac_launch_sparse_retained");
}

void jac_launch_sparse_retained_tp2_local(
    const jacq_half_t* Q, const int32_t* RETAINED_BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
    const jacq_half_t* K_SCALE_PAGES, const jacq_half_t* K_ZERO_PAGES,
    const uint8_t* V_CODE_PAGES, const jacq_half_t* V_SCALE_PAGES,
    const jacq_half_t* V_ZERO_PAGES, const jacq_half_t* K_RESIDUAL_SCRATCH,
    const jacq_half_t* V_RESIDUAL_SCRATCH, int SEQ_LEN, int NUM_RETAINED_PAGES, float* O,
    hipStream_t stream) {
  sparse_v1(kTp2Local, Q, RETAINED_BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
            V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH,
            SEQ_LEN, NUM_RETAINED_PAGES, O, stream, "jac_launch_sparse_retained_tp2_local");
}

static void batched_v1(const jacq_kivi_geometry& x, const jacq_half_t* Q, const int32_t* SEQ_LENS,
                       const int32_t* BLOCK_TABLE, const uint8_t* kc, const jacq_half_t* ks,
                       const jacq_half_t* kz, const uint8_t* vc, const jacq_half_t* vs,
                       const jacq_half_t* vz, const jacq_half_t* kscr, const jacq_half_t* vscr,
                       int NUM_QUERIES, float* O, hipStream_t stream, const char* where) {
  if (NUM_QUERIES < 1) return;  // an empty grid: the reference launch would be a no-op error
  v1_check(v1_decode(x, Q, SEQ_LENS, -1, BLOCK_TABLE, kc, ks, kz, vc, vs, vz, kscr, vscr,
                     NUM_QUERIES, O, stream),
           where);
}

void jac_launch_batched(const jacq_half_t* Q, const int32_t* SEQ_LENS, const int32_t* BLOCK_TABLE,
                        const uint8_t* K_CODE_PAGES, const jacq_half_t* K_SCALE_PAGES,
                        const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                        const jacq_half_t* V_SCALE_PAGES, const jacq_half_t* V_ZERO_PAGES,
                        const jacq_half_t* K_RESIDUAL_SCRATCH,
                        const jacq_half_t* V_RESIDUAL_SCRATCH, int NUM_QUERIES, float* O,
                        hipStream_t stream) {
  batched_v1(kGlobal, Q, SEQ_LENS, BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
             V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH,
             NUM_QUERIES, O, stream, "jac_launch_batched");
}

void jac_launch_batched_tp2_local(const jacq_half_t* Q, const int32_t* SEQ_LENS,
                                  const int32_t* BLOCK_TABLE, const uint8_t* K_CODE_PAGES,
                                  const jacq_half_t* K_SCALE_PAGES,
                                  const jacq_half_t* K_ZERO_PAGES, const uint8_t* V_CODE_PAGES,
                                  const jacq_half_t* V_SCALE_PAGES,
                                  const jacq_half_t* V_ZERO_PAGES,
                                  const jacq_half_t* K_RESIDUAL_SCRATCH,
                                  const jacq_half_t* V_RESIDUAL_SCRATCH, int NUM_QUERIES,
                                  float* O, hipStream_t stream) {
  batched_v1(kTp2Local, Q, SEQ_LENS, BLOCK_TABLE, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
             V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH,
             NUM_QUERIES, O, stream, "jac_launch_batched_tp2_local");
}

static jacq_kivi_geometry writer_geo(int nkv) {
  jacq_kivi_geometry x = kGlobal;
  x.num_kv_heads = nkv;
  x.num_heads = nkv * (kGlobal.num_heads / kGlobal.num_kv_heads);
  return x;
}

void jac_launch_cache_write(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                            jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                            jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                            jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                            const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                            const int32_t* BLOCK_TABLE, int SEQ_LEN, hipStream_t stream) {
  v1_check(run_append(kGlobal, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES,
                      V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, 0,
                      NEW_K, NEW_V, 0, BLOCK_TABLE, 0, nullptr, SEQ_LEN - 1, 1, 1, stream),
           "jac_launch_cache_write");
}

void jac_launch_cache_write_batched(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                                    jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                                    jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                                    jacq_half_t* K_RESIDUAL_SCRATCH,
                                    jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                                    const jacq_half_t* NEW_V, const int32_t* BLOCK_TABLE,
                                    int START_SEQ_LEN, int NUM_NEW, hipStream_t stream) {
  if (NUM_NEW < 1) return;
  v1_check(run_append(kGlobal, K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES, V_CODE_PAGES,
                      V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH, V_RESIDUAL_SCRATCH, 0,
                      NEW_K, NEW_V, 0, BLOCK_TABLE, 0, nullptr, START_SEQ_LEN, NUM_NEW, 1, stream),
           "jac_launch_cache_write_batched");
}

void kivi_cache_write_launch(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                             jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                             jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                             jacq_half_t* K_RESIDUAL_SCRATCH, jacq_half_t* V_RESIDUAL_SCRATCH,
                             const jacq_half_t* NEW_K, const jacq_half_t* NEW_V,
                             const int64_t* SLOT_MAPPING, const int32_t* BLOCK_TABLE, int seq_len,
                             int NKV_RUNTIME, hipStream_t stream) {
  (void)SLOT_MAPPING;  // placement comes from BLOCK_TABLE (source_patch.py:1667-1675)
  if (NKV_RUNTIME < 1) return;
  v1_check(run_append(writer_geo(NKV_RUNTIME), K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
                      V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH,
                      V_RESIDUAL_SCRATCH, 0, NEW_K, NEW_V, 0, BLOCK_TABLE, 0, nullptr, seq_len - 1,
                      1, 1, stream),
           "kivi_cache_write_launch");
}

void kivi_cache_write_batched_launch(uint8_t* K_CODE_PAGES, jacq_half_t* K_SCALE_PAGES,
                                     jacq_half_t* K_ZERO_PAGES, uint8_t* V_CODE_PAGES,
                                     jacq_half_t* V_SCALE_PAGES, jacq_half_t* V_ZERO_PAGES,
                                     jacq_half_t* K_RESIDUAL_SCRATCH,
                                     jacq_half_t* V_RESIDUAL_SCRATCH, const jacq_half_t* NEW_K,
                                     const jacq_half_t* NEW_V, const int64_t* SLOT_MAPPING,
                                     const int32_t* BLOCK_TABLE, int START_SEQ_LEN, int NUM_NEW,
                                     int NKV_RUNTIME, hipStream_t stream) {
  (void)SLOT_MAPPING;
  if (NKV_RUNTIME < 1 || NUM_NEW < 1) return;
  v1_check(run_append(writer_geo(NKV_RUNTIME), K_CODE_PAGES, K_SCALE_PAGES, K_ZERO_PAGES,
                      V_CODE_PAGES, V_SCALE_PAGES, V_ZERO_PAGES, K_RESIDUAL_SCRATCH,
                      V_RESIDUAL_SCRATCH, 0, NEW_K, NEW_V, 0, BLOCK_TABLE, 0, nullptr,
                      START_SEQ_LEN, NUM_NEW, 1, stream),
           "kivi_cache_write_batched_launch");
}

}  // extern "C"

// C++-linkage writer entry points with the reference's parameter types
// (source_patch.py:624-637): the mangled names a hipified reference binding
// links against.  Thin forwards to the C-linkage functions.
void kivi_cache_write_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
                             __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES,
                             __half* V_SCALE_PAGES, __half* V_ZERO_PAGES,
                             __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
                             const __half* NEW_K, const __half* NEW_V,
                             const int64_t* SLOT_MAPPING, const int* BLOCK_TABLE, int seq_len,
                             int NKV_RUNTIME, hipStream_t stream) {
  auto h = [](const __half* p) { return reinterpret_cast<const jacq_half_t*>(p); };
  auto m = [](__half* p) { return reinterpret_cast<jacq_half_t*>(p); };
  kivi_cache_write_launch(K_CODE_PAGES, m(K_SCALE_PAGES), m(K_ZERO_PAGES), V_CODE_PAGES,
                          m(V_SCALE_PAGES), m(V_ZERO_PAGES), m(K_RESIDUAL_SCRATCH),
                          m(V_RESIDUAL_SCRATCH), h(NEW_K), h(NEW_V), SLOT_MAPPING,
                          reinterpret_cast<const int32_t*>(BLOCK_TABLE), seq_len, NKV_RUNTIME,
                          stream);
}

void kivi_cache_write_batched_launch(unsigned char* K_CODE_PAGES, __half* K_SCALE_PAGES,
                                     __half* K_ZERO_PAGES, unsigned char* V_CODE_PAGES,
                                     __half* V_SCALE_PAGES, __half* V_ZERO_PAGES,
                                     __half* K_RESIDUAL_SCRATCH, __half* V_RESIDUAL_SCRATCH,
                                     const __half* NEW_K, const __half* NEW_V,
                                     const int64_t* SLOT_MAPPING, const int* BLOCK_TABLE,
                                     int START_SEQ_LEN, int NUM_NEW, int NKV_RUNTIME,
                                     hipStream_t stream) {
  auto h = [](const __half* p) { return reinterpret_cast<const jacq_half_t*>(p); };
  auto m = [](__half* p) { return reinterpret_cast<jacq_half_t*>(p); };
  kivi_cache_write_batched_launch(K_CODE_PAGES, m(K_SCALE_PAGES), m(K_ZERO_PAGES), V_CODE_PAGES,
                                  m(V_SCALE_PAGES), m(V_ZERO_PAGES), m(K_RESIDUAL_SCRATCH),
                                  m(V_RESIDUAL_SCRATCH), h(NEW_K), h(NEW_V), SLOT_MAPPING,
                                  reinterpret_cast<const int32_t*>(BLOCK_TABLE), START_SEQ_LEN,
                                  NUM_NEW, NKV_RUNTIME, stream);
}
