// libkk runtime: device/stream lifecycle, errors, the bucketed device buffer
// pool, host<->device copies, events, and the host-side descriptor helpers
// (broadcast planning) used by every op.
#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <iterator>
#include <mutex>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "kk_internal.h"

namespace kk {

Context& ctx() {
  static Context c;
  return c;
}

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return KK_OK;
  return set_error(e == hipErrorOutOfMemory ? KK_E_NOMEM : KK_E_HIP,
                   "%s: %s", what, hipGetErrorString(e));
}

int require_ready() {
  if (!ctx().ready) return set_error(KK_E_STATE, "libkk: kk_init() has not been called");
  return KK_OK;
}

int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(KK_E_HIP, "launch of %s failed: %s", kernel, hipGetErrorString(e));
  return KK_OK;
}

// ------------------------------------------------------------ descriptors
int dtype_size(int dt) {
  switch (dt) {
    case KK_F32: case KK_I32: return 4;
    case KK_I8: case KK_U8: case KK_BOOL: return 1;
    case KK_I64: return 8;
    case KK_F16: return 2;
  }
  return 0;
}
bool is_float(int dt) { return dt == KK_F32 || dt == KK_F16; }
bool is_int(int dt) {
  return dt == KK_I8 || dt == KK_U8 || dt == KK_I32 || dt == KK_I64 || dt == KK_BOOL;
}

int64_t numel(const kk_tensor* t) {
  int64_t n = 1;
  for (int i = 0; i < t->rank; ++i) n *= t->shape[i];
  return n;
}

bool is_contiguous(const kk_tensor* t) {
  if (numel(t) == 0) return true;
  int64_t acc = 1;
  for (int i = t->rank - 1; i >= 0; --i) {
    if (t->shape[i] != 1 && t->strides[i] != acc) return false;
    acc *= t->shape[i];
  }
  return true;
}

int check_tensor(const kk_tensor* t, const char* name) {
  if (!t) return set_error(KK_E_ARG, "%s: tensor is NULL", name);
  if (t->rank < 0 || t->rank > KK_MAX_RANK)
    return set_error(KK_E_ARG, "%s: rank %d outside 0..%d", name, t->rank, KK_MAX_RANK);
  if (dtype_size(t->dtype) == 0)
    return set_error(KK_E_ARG, "%s: unknown dtype code %d", name, t->dtype);
  for (int i = 0; i < t->rank; ++i)
    if (t->shape[i] < 0) return set_error(KK_E_ARG, "%s: negative extent", name);
  if (numel(t) > 0 && !t->data) return set_error(KK_E_ARG, "%s: NULL data", name);
  return KK_OK;
}

int make_plan(Plan* p, const kk_tensor* out, const kk_tensor* const* ins, int nins) {
  if (nins + 1 > kMaxOperands) return set_error(KK_E_ARG, "too many operands");
  const int r = out->rank;
  p->nops = nins + 1;
  int64_t dims[KK_MAX_RANK];
  int64_t st[kMaxOperands][KK_MAX_RANK];
  const bool empty = numel(out) == 0;  // nothing is walked: strides are moot
  for (int i = 0; i < r; ++i) {
    dims[i] = out->shape[i];
    st[0][i] = out->strides[i];
    if (!empty && out->shape[i] != 1 && out->strides[i] == 0)
      return set_error(KK_E_ARG, "output must not broadcast (axis %d has stride 0)", i);
  }
  for (int k = 0; k < nins; ++k) {
    const kk_tensor* t = ins[k];
    for (int i = 0; i < r; ++i) st[k + 1][i] = 0;
    if (!t) continue;
    if (t->rank > r)
      return set_error(KK_E_ARG, "operand %d has rank %d > output rank %d", k, t->rank, r);
    const int pad = r - t->rank;
    for (int i = 0; i < t->rank; ++i) {
      const int64_t d = t->shape[i], od = out->shape[pad + i];
      if (d == od) {
        st[k + 1][pad + i] = t->strides[i];
      } else if (d == 1) {
        st[k + 1][pad + i] = 0;  // broadcast: never advance along this axis
      } else {
        return set_error(KK_E_ARG, "operand %d extent %lld does not broadcast to %lld (axis %d)",
                         k, (long long)d, (long long)od, pad + i);
      }
    }
  }
  // Drop unit axes.
  int n = 0;
  p->n = 1;
  for (int i = 0; i < r; ++i) {
    p->n *= dims[i];
    if (dims[i] == 1) continue;
    p->dims[n] = dims[i];
    for (int k = 0; k < p->nops; ++k) p->st[k][n] = st[k][i];
    ++n;
  }
  // Merge axis i into i-1 when every operand's outer stride equals its inner
  // stride times the inner extent (broadcast axes satisfy 0 == 0 * d).
  for (int i = n - 1; i > 0; --i) {
    bool ok = true;
    for (int k = 0; k < p->nops; ++k)
      if (p->st[k][i - 1] != p->st[k][i] * p->dims[i]) { ok = false; break; }
    if (!ok) continue;
    p->dims[i - 1] *= p->dims[i];
    for (int k = 0; k < p->nops; ++k) p->st[k][i - 1] = p->st[k][i];
    for (int j = i; j < n - 1; ++j) {
      p->dims[j] = p->dims[j + 1];
      for (int k = 0; k < p->nops; ++k) p->st[k][j] = p->st[k][j + 1];
    }
    --n;
  }
  if (n == 0) {
    p->dims[0] = 1;
    for (int k = 0; k < p->nops; ++k) p->st[k][0] = 0;
    n = 1;
  }
  p->rank = n;
  return KK_OK;
}

int make_dequant(Dequant* d, const kk_tensor* w, const kk_tensor* scale,
                 const kk_tensor* zp, int64_t count, const char* who) {
  *d = Dequant();
  const bool quant = (w->dtype == KK_I8 || w->dtype == KK_U8);
  if (!quant) {
    if (w->dtype != KK_F32 && w->dtype != KK_F16)
      return set_error(KK_E_ARG, "%s: weight dtype %d unsupported", who, w->dtype);
    if (scale || zp)
      return set_error(KK_E_ARG, "%s: scale/zero point given for a float weight", who);
    return KK_OK;
  }
  if (!scale) return set_error(KK_E_ARG, "%s: int8/uint8 weight needs a scale", who);
  KK_TRY(check_tensor(scale, "w_scale"));
  if (!is_float(scale->dtype)) return set_error(KK_E_ARG, "%s: scale must be f32/f16", who);
  const int64_t ns = numel(scale);
  if (ns != 1 && ns != count)
    return set_error(KK_E_ARG, "%s: scale has %lld elements, expected 1 or %lld", who,
                     (long long)ns, (long long)count);
  if (ns > 1 && !is_contiguous(scale))
    return set_error(KK_E_ARG, "%s: per-column scale must be contiguous", who);
  d->scale = scale->data;
  d->scale_dt = scale->dtype;
  d->scale_stride = ns > 1 ? 1 : 0;
  if (zp) {
    KK_TRY(check_tensor(zp, "w_zp"));
    if (!(zp->dtype == KK_I8 || zp->dtype == KK_U8 || zp->dtype == KK_I32))
      return set_error(KK_E_ARG, "%s: zero point must be int8/uint8/int32", who);
    const int64_t nz = numel(zp);
    if (nz != 1 && nz != count)
      return set_error(KK_E_ARG, "%s: zero point has %lld elements, expected 1 or %lld", who,
                       (long long)nz, (long long)count);
    if (nz > 1 && !is_contiguous(zp))
      return set_error(KK_E_ARG, "%s: per-column zero point must be contiguous", who);
    d->zp = zp->data;
    d->zp_dt = zp->dtype;
    d->zp_stride = nz > 1 ? 1 : 0;
  }
  d->active = true;
  return KK_OK;
}

// ------------------------------------------------------------------- pool
// Buckets keep four significant bits of the size with a 256-byte floor, so a
// buffer is less than 12.5% larger than asked and runs of different lengths
// reuse each other's buffers (the rounding rule of executor.gd:206-216).
static size_t bucket_size(size_t nbytes) {
  size_t size = std::max<size_t>(256, (nbytes + 255) & ~size_t(255));
  if (size <= 4096) return size;
  int shift = 0;
  for (size_t v = size; v > 15; v >>= 1) ++shift;
  const size_t gran = size_t(1) << shift;
  return (size + gran - 1) & ~(gran - 1);
}

struct Pool {
  std::mutex mu;
  std::unordered_map<void*, size_t> live;      // every buffer we own -> bucket
  std::unordered_set<void*> in_pool;           // subset of `live` that is free
  std::unordered_map<size_t, std::vector<void*>> free_lists;
  size_t live_bytes = 0;    // bytes handed out to callers
  size_t pooled_bytes = 0;  // bytes sitting in free lists
  size_t peak_live = 0;
};
static Pool& pool() {
  static Pool* p = new Pool();  // leaked on purpose: outlives static dtors
  return *p;
}

static void pool_release_all() {
  Pool& p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  for (auto& kv : p.live) (void)hipFree(kv.first);
  p.live.clear();
  p.in_pool.clear();
  p.free_lists.clear();
  p.live_bytes = p.pooled_bytes = 0;
}

// ------------------------------------------------------------ leaf sums
// Which tensor a convolution's leaf sums were formed from (an InstanceNorm
// takes them only for that tensor); forgotten when either buffer is freed.
struct LeafRec {
  const void* x;
  int64_t rows, T;
};
static std::mutex g_leaf_mu;
static std::unordered_map<const void*, LeafRec>& leaf_recs() {
  static auto* m = new std::unordered_map<const void*, LeafRec>();
  return *m;
}

void leaf_record(const void* leaf, const void* x, int64_t rows, int64_t T) {
  std::lock_guard<std::mutex> lk(g_leaf_mu);
  leaf_recs()[leaf] = LeafRec{x, rows, T};
}

bool leaf_matches(const void* leaf, const void* x, int64_t rows, int64_t T) {
  std::lock_guard<std::mutex> lk(g_leaf_mu);
  auto it = leaf_recs().find(leaf);
  return it != leaf_recs().end() && it->second.x == x && it->second.rows == rows &&
         it->second.T == T;
}

static void leaf_forget(const void* p) {
  std::lock_guard<std::mutex> lk(g_leaf_mu);
  auto& m = leaf_recs();
  if (m.empty()) return;
  m.erase(p);
  for (auto it = m.begin(); it != m.end();)
    it = it->second.x == p ? m.erase(it) : std::next(it);
}

// Every record whose leaf buffer or x lies in [base, base + bytes).
static void leaf_forget_range(const char* base, size_t bytes) {
  std::lock_guard<std::mutex> lk(g_leaf_mu);
  auto& m = leaf_recs();
  auto in = [base, bytes](const void* q) {
    const char* c = static_cast<const char*>(q);
    return c >= base && c < base + bytes;
  };
  for (auto it = m.begin(); it != m.end();)
    it = in(it->first) || in(it->second.x) ? m.erase(it) : std::next(it);
}

// ---------------------------------------------------------- graph arenas
// Device memory owned by a graph recorded with kk_graph_begin_arena.  While
// it is recorded, kk_alloc hands out the arena's blocks (the pool's buckets,
// a free list per bucket, so that a block freed by one op is reused by a
// later one exactly as it would be in the pool: the recorded kernels run in
// recording order), and a pool buffer freed by an op is held by the graph
// instead of returning to the pool, since every replay reads it again.
// Arena blocks are released only with the graph (kk_free of one is then a
// no-op); held buffers go back to the pool at the same time.
struct Arena {
  char* base = nullptr;
  size_t bytes = 0, top = 0;
  std::unordered_map<void*, size_t> size_of;  // every block handed out -> bucket
  std::unordered_map<size_t, std::vector<void*>> free_lists;
  std::vector<void*> held;  // pool buffers freed while recording
  bool owns(const void* p) const {
    const char* c = static_cast<const char*>(p);
    return c >= base && c < base + bytes;
  }
};
static Arena* g_rec_arena = nullptr;   // the arena of the graph being recorded
static Arena* g_dead_arena = nullptr;  // a recording kk_graph_end could not make a graph of

static int arena_alloc(Arena& a, size_t nbytes, void** dptr) {
  const size_t size = bucket_size(nbytes);
  auto it = a.free_lists.find(size);
  if (it != a.free_lists.end() && !it->second.empty()) {
    *dptr = it->second.back();
    it->second.pop_back();
    return KK_OK;
  }
  if (a.top + size > a.bytes)
    return set_error(KK_E_NOMEM, "graph arena exhausted: %zu of %zu bytes in use, %zu more asked",
                     a.top, a.bytes, size);
  void* q = a.base + a.top;
  a.top += size;
  a.size_of[q] = size;
  *dptr = q;
  return KK_OK;
}

// Releases an arena whose graph has gone (or was never made): its blocks,
// and its held buffers back to the pool.  The stream must not be running
// work that reads them.
static void arena_release(Arena* a) {
  if (!a) return;
  Pool& p = pool();
  {
    std::lock_guard<std::mutex> lk(p.mu);
    for (void* q : a->held) {
      auto it = p.live.find(q);
      if (it == p.live.end() || p.in_pool.count(q)) continue;
      conv_i8_forget_pack(q);
      convh_forget_pack(q);
      gemm_forget_pack(q);
      i8_forget_pack(q);
      p.in_pool.insert(q);
      p.free_lists[it->second].push_back(q);
      p.pooled_bytes += it->second;
      p.live_bytes -= it->second;
    }
  }
  if (a->base) {
    leaf_forget_range(a->base, a->bytes);
    (void)hipFree(a->base);
  }
  delete a;
}

// ---------------------------------------------------------------- uploads
// kk_upload never waits for the stream.  Up to kUploadArgBytes travel inside
// the arguments of a one-block copy kernel (kernel arguments are captured at
// launch); larger uploads are staged in a pinned ring and copied with
// hipMemcpyAsync, each staged range guarded by an event until its copy has
// run.  Uploads larger than a quarter of the ring are copied synchronously.
constexpr size_t kUploadArgBytes = 2048;
constexpr size_t kStageBytes = size_t(64) << 20;

struct UploadArgs {
  uint8_t* dst;
  uint32_t n;
  uint8_t data[kUploadArgBytes];
};

__global__ void upload_small_kernel(UploadArgs a) {
  for (uint32_t i = threadIdx.x; i < a.n; i += blockDim.x) a.dst[i] = a.data[i];
}

struct Staged {
  size_t begin, end;
  hipEvent_t done;
};
struct Staging {
  char* ring = nullptr;
  size_t head = 0;
  std::vector<Staged> inflight;
  std::vector<hipEvent_t> spare;
};
static Staging& staging() {
  static Staging* s = new Staging();  // leaked on purpose: outlives static dtors
  return *s;
}

static int stage_upload(void* dst, const void* src, size_t bytes) {
  Staging& S = staging();
  if (!S.ring) KK_HIP(hipHostMalloc(reinterpret_cast<void**>(&S.ring), kStageBytes,
                                    hipHostMallocDefault));
  const size_t len = (bytes + 255) & ~size_t(255);
  if (S.head + len > kStageBytes) S.head = 0;
  const size_t b = S.head, e = b + len;
  // Wait for (and retire) staged copies that overlap [b, e) or have finished.
  for (size_t k = 0; k < S.inflight.size();) {
    Staged& st = S.inflight[k];
    const bool overlap = st.begin < e && b < st.end;
    if (overlap) KK_HIP(hipEventSynchronize(st.done));
    if (overlap || hipEventQuery(st.done) == hipSuccess) {
      S.spare.push_back(st.done);
      S.inflight[k] = S.inflight.back();
      S.inflight.pop_back();
    } else {
      ++k;
    }
  }
  std::memcpy(S.ring + b, src, bytes);
  KK_HIP(hipMemcpyAsync(dst, S.ring + b, bytes, hipMemcpyHostToDevice, ctx().stream));
  hipEvent_t ev;
  if (!S.spare.empty()) {
    ev = S.spare.back();
    S.spare.pop_back();
  } else {
    KK_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  KK_HIP(hipEventRecord(ev, ctx().stream));
  S.inflight.push_back(Staged{b, e, ev});
  S.head = e;
  return KK_OK;
}

static void staging_release() {
  Staging& S = staging();
  for (auto& st : S.inflight) S.spare.push_back(st.done);
  S.inflight.clear();
  for (hipEvent_t ev : S.spare) (void)hipEventDestroy(ev);
  S.spare.clear();
  if (S.ring) (void)hipHostFree(S.ring);
  S.ring = nullptr;
  S.head = 0;
}

// ----------------------------------------------------------------- events
static hipEvent_t g_events[KK_MAX_EVENTS];
static bool g_event_made[KK_MAX_EVENTS];

// ----------------------------------------------------------------- graphs
struct GraphSlot {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  Arena* arena = nullptr;
};
static std::vector<GraphSlot>& graphs() {
  static std::vector<GraphSlot>* g = new std::vector<GraphSlot>();
  return *g;
}

// The arena (of the graph being recorded or of a recorded one) holding p.
static Arena* arena_of(const void* p) {
  if (g_rec_arena && g_rec_arena->owns(p)) return g_rec_arena;
  if (g_dead_arena && g_dead_arena->owns(p)) return g_dead_arena;
  for (auto& s : graphs())
    if (s.arena && s.arena->owns(p)) return s.arena;
  return nullptr;
}

static int not_capturing(const char* who) {
  if (ctx().capturing)
    return set_error(KK_E_STATE, "%s is not allowed while a graph is being recorded", who);
  return KK_OK;
}

static void destroy_graphs() {
  for (auto& s : graphs()) {
    if (s.exec) (void)hipGraphExecDestroy(s.exec);
    if (s.graph) (void)hipGraphDestroy(s.graph);
    arena_release(s.arena);
    s = GraphSlot();
  }
}

// Ends a recording that will not become a graph.
static void abandon_recording() {
  Context& c = ctx();
  if (!c.capturing) return;
  hipGraph_t g = nullptr;
  (void)hipStreamEndCapture(c.stream, &g);
  if (g) (void)hipGraphDestroy(g);
  (void)hipGetLastError();
  c.capturing = false;
  arena_release(g_rec_arena);  // nothing recorded into it has run
  g_rec_arena = nullptr;
}

// kk_graph_end's failures keep the recording's arena (the caller may still
// hold its blocks) until kk_graph_abort.
static void keep_dead_arena(Arena* a) {
  arena_release(g_dead_arena);
  g_dead_arena = a;
}

}  // namespace kk

using namespace kk;

extern "C" {

const char* kk_last_error(void) { return g_last_error.c_str(); }

int kk_device_count(int* count) {
  if (!count) return set_error(KK_E_ARG, "count is NULL");
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) n = 0;
  *count = n;
  return KK_OK;
}

int kk_init(int device) {
  Context& c = ctx();
  if (c.ready) {
    if (c.device == device) return KK_OK;
    return set_error(KK_E_STATE, "libkk already initialised on device %d", c.device);
  }
  int n = 0;
  KK_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n)
    return set_error(KK_E_ARG, "device %d not present (%d visible)", device, n);
  KK_HIP(hipSetDevice(device));
  KK_HIP(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
  hipDeviceProp_t prop;
  KK_HIP(hipGetDeviceProperties(&prop, device));
  c.num_cus = prop.multiProcessorCount;
  KK_HIP(hipMalloc(reinterpret_cast<void**>(&c.row_counters),
                   sizeof(int) * (kRowCounters + kFlagSlots)));
  KK_HIP(hipMemset(c.row_counters, 0, sizeof(int) * (kRowCounters + kFlagSlots)));
  KK_HIP(hipMalloc(&c.scratch, kScratchBytes));
  KK_TRY(conv_i8_scratch_setup(device));
  c.device = device;
  c.ready = true;
  return KK_OK;
}

int kk_shutdown(void) {
  Context& c = ctx();
  if (!c.ready) return KK_OK;
  abandon_recording();
  (void)hipStreamSynchronize(c.stream);
  destroy_graphs();
  arena_release(g_dead_arena);
  g_dead_arena = nullptr;
  pool_release_all();
  staging_release();
  if (c.row_counters) { (void)hipFree(c.row_counters); c.row_counters = nullptr; }
  if (c.scratch) { (void)hipFree(c.scratch); c.scratch = nullptr; }
  for (int i = 0; i < KK_MAX_EVENTS; ++i)
    if (g_event_made[i]) { (void)hipEventDestroy(g_events[i]); g_event_made[i] = false; }
  (void)hipStreamDestroy(c.stream);
  c.stream = nullptr;
  c.ready = false;
  c.device = -1;
  return KK_OK;
}

int kk_sync(void) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_sync"));
  KK_HIP(hipStreamSynchronize(ctx().stream));
  return KK_OK;
}

int kk_alloc(size_t bytes, void** dptr) {
  KK_TRY(require_ready());
  if (!dptr) return set_error(KK_E_ARG, "dptr is NULL");
  if (ctx().capturing) {
    if (!g_rec_arena)
      return set_error(KK_E_STATE, "kk_alloc is not allowed while a graph is being recorded "
                                   "without an arena (kk_graph_begin_arena)");
    return arena_alloc(*g_rec_arena, bytes, dptr);
  }
  const size_t size = bucket_size(bytes);
  Pool& p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.free_lists.find(size);
  if (it != p.free_lists.end() && !it->second.empty()) {
    void* q = it->second.back();
    it->second.pop_back();
    p.in_pool.erase(q);
    p.pooled_bytes -= size;
    p.live_bytes += size;
    p.peak_live = std::max(p.peak_live, p.live_bytes);
    *dptr = q;
    return KK_OK;
  }
  void* q = nullptr;
  hipError_t e = hipMalloc(&q, size);
  if (e != hipSuccess) {
    // Give the pooled memory back to the device and try once more.  Pooled
    // buffers may still be read by enqueued work, so drain the stream first.
    (void)hipStreamSynchronize(ctx().stream);
    for (auto& kv : p.free_lists)
      for (void* f : kv.second) { (void)hipFree(f); p.live.erase(f); p.in_pool.erase(f); }
    p.free_lists.clear();
    p.pooled_bytes = 0;
    (void)hipGetLastError();
    e = hipMalloc(&q, size);
    if (e != hipSuccess)
      return set_error(KK_E_NOMEM, "hipMalloc(%zu) failed: %s", size, hipGetErrorString(e));
  }
  p.live[q] = size;
  p.live_bytes += size;
  p.peak_live = std::max(p.peak_live, p.live_bytes);
  *dptr = q;
  return KK_OK;
}

int kk_free(void* dptr) {
  if (!dptr) return KK_OK;
  KK_TRY(require_ready());
  leaf_forget(dptr);
  if (Arena* a = arena_of(dptr)) {
    if (a != g_rec_arena) return KK_OK;  // a recorded graph's: released with it
    auto sz = a->size_of.find(dptr);
    if (sz == a->size_of.end())
      return set_error(KK_E_STATE, "kk_free: %p is not a block of the graph arena", dptr);
    a->free_lists[sz->second].push_back(dptr);
    return KK_OK;
  }
  Pool& p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  auto it = p.live.find(dptr);
  if (it == p.live.end())
    return set_error(KK_E_STATE, "kk_free: %p was not allocated by kk_alloc", dptr);
  if (p.in_pool.count(dptr))
    return set_error(KK_E_STATE, "kk_free: %p freed twice", dptr);
  if (g_rec_arena) {
    // read again by every replay of the graph being recorded
    for (void* q : g_rec_arena->held)
      if (q == dptr) return set_error(KK_E_STATE, "kk_free: %p freed twice", dptr);
    g_rec_arena->held.push_back(dptr);
    return KK_OK;
  }
  // Work already enqueued on the stream that reads this buffer stays
  // ordered before any later reuse, because every op runs on one stream.
  p.in_pool.insert(dptr);
  p.free_lists[it->second].push_back(dptr);
  conv_i8_forget_pack(dptr);
  convh_forget_pack(dptr);
  gemm_forget_pack(dptr);
  i8_forget_pack(dptr);
  p.pooled_bytes += it->second;
  p.live_bytes -= it->second;
  return KK_OK;
}

int kk_pool_stats(size_t* live_bytes, size_t* pooled_bytes, size_t* peak_live_bytes) {
  Pool& p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  if (live_bytes) *live_bytes = p.live_bytes;
  if (pooled_bytes) *pooled_bytes = p.pooled_bytes;
  if (peak_live_bytes) *peak_live_bytes = p.peak_live;
  return KK_OK;
}

int kk_pool_trim(size_t budget_bytes) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_pool_trim"));
  KK_HIP(hipStreamSynchronize(ctx().stream));
  Pool& p = pool();
  std::lock_guard<std::mutex> lk(p.mu);
  // Free the largest buckets first until the pool fits the budget.
  std::vector<size_t> sizes;
  for (auto& kv : p.free_lists) sizes.push_back(kv.first);
  std::sort(sizes.rbegin(), sizes.rend());
  for (size_t s : sizes) {
    auto& lst = p.free_lists[s];
    while (!lst.empty() && p.pooled_bytes > budget_bytes) {
      void* q = lst.back();
      lst.pop_back();
      p.in_pool.erase(q);
      p.live.erase(q);
      p.pooled_bytes -= s;
      KK_HIP(hipFree(q));
    }
  }
  return KK_OK;
}

int kk_upload(void* dst, const void* src, size_t bytes) {
  KK_TRY(require_ready());
  if (ctx().capturing && !g_rec_arena)
    return set_error(KK_E_STATE, "kk_upload is not allowed while a graph is being recorded "
                                 "without an arena (kk_graph_begin_arena)");
  if (!bytes) return KK_OK;
  if (!dst || !src) return set_error(KK_E_ARG, "kk_upload: NULL pointer");
  if (ctx().capturing) {
    // Recorded with an arena: the bytes become arguments of copy kernels in
    // the graph (a host staging buffer would be read again, changed, by
    // every replay), kUploadArgBytes a kernel.
    for (size_t at = 0; at < bytes; at += kUploadArgBytes) {
      UploadArgs a;
      a.dst = static_cast<uint8_t*>(dst) + at;
      a.n = static_cast<uint32_t>(std::min(kUploadArgBytes, bytes - at));
      std::memcpy(a.data, static_cast<const uint8_t*>(src) + at, a.n);
      KK_LAUNCH(upload_small_kernel, dim3(1), dim3(256), 0, ctx().stream, a);
      KK_TRY(check_launch("upload_small_kernel"));
    }
    return KK_OK;
  }
  // The host buffer belongs to the caller, who may release it on return: its
  // bytes are captured (kernel arguments or the staging ring) before that.
  if (bytes <= kUploadArgBytes) {
    UploadArgs a;
    a.dst = static_cast<uint8_t*>(dst);
    a.n = static_cast<uint32_t>(bytes);
    std::memcpy(a.data, src, bytes);
    KK_LAUNCH(upload_small_kernel, dim3(1), dim3(256), 0, ctx().stream, a);
    return check_launch("upload_small_kernel");
  }
  if (bytes <= kStageBytes / 4) return stage_upload(dst, src, bytes);
  KK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx().stream));
  KK_HIP(hipStreamSynchronize(ctx().stream));
  return KK_OK;
}

int kk_download(void* dst, const void* src, size_t bytes) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_download"));
  if (!bytes) return KK_OK;
  if (!dst || !src) return set_error(KK_E_ARG, "kk_download: NULL pointer");
  KK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx().stream));
  KK_HIP(hipStreamSynchronize(ctx().stream));
  return KK_OK;
}

int kk_event_record(int slot) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_event_record"));
  if (slot < 0 || slot >= KK_MAX_EVENTS) return set_error(KK_E_ARG, "event slot %d", slot);
  if (!g_event_made[slot]) {
    KK_HIP(hipEventCreate(&g_events[slot]));
    g_event_made[slot] = true;
  }
  KK_HIP(hipEventRecord(g_events[slot], ctx().stream));
  return KK_OK;
}

int kk_event_elapsed(int a, int b, float* ms) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_event_elapsed"));
  if (a < 0 || a >= KK_MAX_EVENTS || b < 0 || b >= KK_MAX_EVENTS || !g_event_made[a] ||
      !g_event_made[b] || !ms)
    return set_error(KK_E_ARG, "kk_event_elapsed: bad slots %d/%d", a, b);
  KK_HIP(hipEventSynchronize(g_events[b]));
  KK_HIP(hipEventElapsedTime(ms, g_events[a], g_events[b]));
  return KK_OK;
}

int kk_graph_begin(void) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_graph_begin"));
  // Thread-local mode: HIP itself refuses unsafe calls (hipMalloc) made by
  // this thread while recording.
  KK_HIP(hipStreamBeginCapture(ctx().stream, hipStreamCaptureModeThreadLocal));
  ctx().capturing = true;
  return KK_OK;
}

int kk_graph_begin_arena(size_t arena_bytes) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_graph_begin_arena"));
  if (arena_bytes == 0) return set_error(KK_E_ARG, "kk_graph_begin_arena: empty arena");
  Arena* a = new Arena();
  a->bytes = (arena_bytes + 255) & ~size_t(255);
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&a->base), a->bytes);
  if (e != hipSuccess) {
    delete a;
    (void)hipGetLastError();
    return set_error(KK_E_NOMEM, "kk_graph_begin_arena: hipMalloc(%zu) failed: %s", arena_bytes,
                     hipGetErrorString(e));
  }
  e = hipStreamBeginCapture(ctx().stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    arena_release(a);
    return check_hip(e, "hipStreamBeginCapture");
  }
  g_rec_arena = a;
  ctx().capturing = true;
  return KK_OK;
}

int kk_graph_abort(void) {
  KK_TRY(require_ready());
  if (ctx().capturing) {
    abandon_recording();
  } else if (g_dead_arena) {
    arena_release(g_dead_arena);
    g_dead_arena = nullptr;
  } else {
    return set_error(KK_E_STATE, "kk_graph_abort without a recording");
  }
  return KK_OK;
}

int kk_graph_end(int* graph_id) {
  KK_TRY(require_ready());
  if (!ctx().capturing) return set_error(KK_E_STATE, "kk_graph_end without kk_graph_begin");
  if (!graph_id) {
    abandon_recording();
    return set_error(KK_E_ARG, "graph_id is NULL");
  }
  ctx().capturing = false;
  GraphSlot s;
  s.arena = g_rec_arena;
  g_rec_arena = nullptr;
  hipError_t e = hipStreamEndCapture(ctx().stream, &s.graph);
  if (e != hipSuccess) {
    if (s.graph) (void)hipGraphDestroy(s.graph);
    keep_dead_arena(s.arena);
    return check_hip(e, "hipStreamEndCapture");
  }
  e = hipGraphInstantiate(&s.exec, s.graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(s.graph);
    keep_dead_arena(s.arena);
    return check_hip(e, "hipGraphInstantiate");
  }
  // Uploaded now, so that the first launch costs what later ones do.
  e = hipGraphUpload(s.exec, ctx().stream);
  if (e != hipSuccess) {
    (void)hipGraphExecDestroy(s.exec);
    (void)hipGraphDestroy(s.graph);
    keep_dead_arena(s.arena);
    return check_hip(e, "hipGraphUpload");
  }
  auto& g = graphs();
  for (size_t i = 0; i < g.size(); ++i)
    if (!g[i].exec) { g[i] = s; *graph_id = static_cast<int>(i); return KK_OK; }
  g.push_back(s);
  *graph_id = static_cast<int>(g.size() - 1);
  return KK_OK;
}

int kk_graph_launch(int graph_id) {
  KK_TRY(require_ready());
  KK_TRY(not_capturing("kk_graph_launch"));
  auto& g = graphs();
  if (graph_id < 0 || graph_id >= static_cast<int>(g.size()) || !g[graph_id].exec)
    return set_error(KK_E_ARG, "kk_graph_launch: no graph %d", graph_id);
  KK_HIP(hipGraphLaunch(g[graph_id].exec, ctx().stream));
  return KK_OK;
}

int kk_graph_destroy(int graph_id) {
  KK_TRY(require_ready());
  auto& g = graphs();
  if (graph_id < 0 || graph_id >= static_cast<int>(g.size()) || !g[graph_id].exec)
    return set_error(KK_E_ARG, "kk_graph_destroy: no graph %d", graph_id);
  // A launched graph may still be running.
  KK_HIP(hipStreamSynchronize(ctx().stream));
  (void)hipGraphExecDestroy(g[graph_id].exec);
  (void)hipGraphDestroy(g[graph_id].graph);
  arena_release(g[graph_id].arena);
  g[graph_id] = GraphSlot();
  return KK_OK;
}

int kk_graph_nodes(int graph_id, int64_t* nodes) {
  KK_TRY(require_ready());
  auto& g = graphs();
  if (graph_id < 0 || graph_id >= static_cast<int>(g.size()) || !g[graph_id].exec || !nodes)
    return set_error(KK_E_ARG, "kk_graph_nodes: no graph %d", graph_id);
  size_t n = 0;
  KK_HIP(hipGraphGetNodes(g[graph_id].graph, nullptr, &n));
  *nodes = static_cast<int64_t>(n);
  return KK_OK;
}

int kk_dispatch_count(uint64_t* dispatches) {
  KK_TRY(require_ready());
  if (!dispatches) return set_error(KK_E_ARG, "kk_dispatch_count: NULL output");
  *dispatches = ctx().dispatches;
  return KK_OK;
}

}  // extern "C"
