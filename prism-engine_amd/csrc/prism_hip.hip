// prism_hip.hip -- C ABI of the MI355X palettized-LUT contraction
// (declarations and contract: include/prism_hip.h).
//
// Host side: argument validation, device staging for host-pointer calls,
// kernel selection per shape, and the keyed HipBackend that mirrors the
// reference's MetalBackend (src/lut/engine_impl.rs:31-490).  There is no
// CPU fallback: every failure is returned as a negative code with text.
#include "prism_hip.h"

#include <cxxabi.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>
#include <unordered_map>
#include <unordered_set>

#include "gemm_kernels.hpp"
#include "gemv_kernels.hpp"
#include "gemv_tile.hpp"
#include "gemv_lpr.hpp"
#include "gemv_mfma.hpp"
#include "measure_kernels.hpp"
#include "palette_kernels.hpp"
#include "step_kernels.hpp"

#define PRISM_HIP_VERSION "prism_hip 0.1 gfx950"

// Device memory of weights: one hipMalloc per chunk instead of one per
// tensor.  A context carves its uploads, 256-byte aligned and in upload
// order, out of its current chunk (8 MB first, doubling up to 64 MB);
// tensors over 16 MB get a chunk of their own.  A chunk is freed when the
// last weight in it is freed and no context carves from it any more, so
// weights outlive their context as before and a freed weight's bytes are
// reused only with its whole chunk.  MI355X: the 168 per-layer hipMallocs of
// a Qwen2.5-0.5B model take 2.3-5.4 ms and their hipFrees 17-20 ms.
struct WeightChunk {
  uint8_t* base = nullptr;
  size_t size = 0, used = 0;
  int device = 0;
  std::atomic<int> refs{0};  // weights in the chunk, plus one while a context carves from it
};

struct prism_hip_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cu = 256;
  size_t lds_max = 65536;  // dynamic + static LDS bytes one workgroup may use
  void* d_stage = nullptr;
  size_t stage_bytes = 0;
  // Stream-ordered pool for per-call device scratch (split-K partials),
  // created on first use; it keeps what it has allocated, so a call after
  // the first reuses memory instead of allocating.
  hipMemPool_t pool = nullptr;
  // This device's address of the static split-K scratch (looked up on the
  // first prism_hip_gemm_dev_noalloc).
  float* scratch = nullptr;
  // Host uploads: a ring of pinned staging buffers (created on first use),
  // each with the event of the last copy out of it, and a device buffer for
  // split-block payloads on their way to the GI layout.
  static constexpr int kRingSlots = 4;
  static constexpr size_t kRingSlotBytes = (size_t)16 << 20;
  void* ring[kRingSlots] = {};
  hipEvent_t ring_done[kRingSlots] = {};
  int ring_next = 0;
  void* d_upload = nullptr;
  size_t upload_bytes = 0;
  // The chunk uploads are carved from (holds one reference) and the size of
  // the next one.
  WeightChunk* carve = nullptr;
  size_t next_chunk = (size_t)8 << 20;
  std::string err;
  // Weights uploaded through this context; destroying the context orphans
  // them (w->ctx = nullptr) so a later prism_hip_weight_free stays valid.
  std::unordered_set<prism_hip_weight*> weights;
  // Decode-step models created on this context, orphaned the same way.
  std::unordered_set<prism_hip_model*> models;
  // Host functions of the kernels the last compute call launched, in
  // order, and their names once asked for (prism_hip_last_kernels).
  std::vector<const void*> launched;
  std::string kernels;
};

namespace prism {

// The launch log of the compute call running on this thread (NULL outside
// one): every dispatch site appends the kernel it launches.
thread_local std::vector<const void*>* g_launch_log = nullptr;

void note_launch(const void* fn) {
  if (g_launch_log) g_launch_log->push_back(fn);
}

}  // namespace prism

// hipLaunchKernelGGL that records the kernel (KERNEL as for
// hipLaunchKernelGGL: a template-id in parentheses).
#define PRISM_LAUNCH(KERNEL, ...)                                 \
  do {                                                            \
    prism::note_launch(reinterpret_cast<const void*>(&KERNEL));   \
    hipLaunchKernelGGL(KERNEL, __VA_ARGS__);                      \
  } while (0)

// hipLaunchKernel that records the kernel.
static hipError_t launch_fn(const void* fn, dim3 grid, dim3 block, void** args, size_t lds, hipStream_t st) {
  prism::note_launch(fn);
  return hipLaunchKernel(fn, grid, block, args, lds, st);
}

// For the length of one compute call: clears the context's launch log and
// makes it the thread's.
struct LaunchLog {
  std::vector<const void*>* prev;
  explicit LaunchLog(prism_hip_ctx* ctx) : prev(prism::g_launch_log) {
    ctx->launched.clear();
    ctx->kernels.clear();
    prism::g_launch_log = &ctx->launched;
  }
  ~LaunchLog() { prism::g_launch_log = prev; }
};

// Defined with prism_hip_model (model_step.hpp): forget the context.
static void model_detach(prism_hip_model* m);

// A weight's device copy is either the split-block payload as uploaded or,
// for 4-bit matrices the lane-per-row GEMV covers in one round of row groups,
// the GI layout (gemv_lpr.hpp: the same bytes regrouped per group of gi
// rows, each group's LUTs before its index chunks).  Kernels over GI take
// the base pointer as both their LUT and their index pointer.
struct prism_hip_weight {
  prism_hip_ctx* ctx = nullptr;
  int device = 0;
  uint32_t dim_m = 0, dim_n = 0, bits = 0, layout = 0;
  size_t bytes = 0;  // payload bytes as uploaded (split-block)
  uint32_t gi = 0;  // GI layout: rows per group; 0: split-block
  uint8_t* d = nullptr;
  WeightChunk* chunk = nullptr;  // the device memory d lies in
  const uint8_t* lut() const { return d; }
  const uint8_t* idx() const { return gi ? d : d + (size_t)dim_m * (2u << bits); }
};

// Split-K partials of prism_hip_gemm_dev_noalloc, the GEMM entry point that
// allocates nothing: one array on each GPU, held until the process ends.
// 64 MiB bounds every split the GEMM dispatch makes on a 256-CU MI355X (at
// most one 256 x 256 fp32 partial tile per CU).  In host code `scratch` is a
// host-side stand-in, never a device address: device_scratch() looks up each
// device's copy once, with that device current, and only that address is
// passed to kernels.
constexpr size_t kScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

namespace {

thread_local std::string g_create_err;

// This device's address of `scratch` (the device is current), looked up
// once per device on the first no-alloc call that needs it.
hipError_t device_scratch(int device, float** out) {
  static std::mutex mu;
  static float* addr[64] = {};
  if (device < 0 || device >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[device] = static_cast<float*>(p);
  }
  *out = addr[device];
  return hipSuccess;
}

int fail(prism_hip_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf;
  return code;
}

#define HIP_TRY(ctx, expr)                                                                          \
  do {                                                                                              \
    hipError_t e_ = (expr);                                                                         \
    if (e_ != hipSuccess)                                                                           \
      return fail((ctx), PRISM_HIP_ERR_DEVICE, "%s failed: %s", #expr, hipGetErrorString(e_));     \
  } while (0)

size_t expected_bytes(uint32_t dm, uint32_t dn, uint32_t bits) {
  const size_t lut = (size_t)dm * (2u << bits);
  const size_t idx = (bits == 4) ? (size_t)dm * (dn / 2) : (size_t)dm * dn;
  return lut + idx;
}

int check_shape(prism_hip_ctx* ctx, uint32_t dm, uint32_t dn, uint32_t bits, uint32_t layout, size_t bytes) {
  if (bits != 4 && bits != 8) return fail(ctx, PRISM_HIP_ERR_BITS, "bits must be 4 or 8, got %u", bits);
  if (layout != PRISM_HIP_LAYOUT_SPLIT_BLOCK) return fail(ctx, PRISM_HIP_ERR_LAYOUT, "unknown layout %u", layout);
  if (dm == 0 || dn == 0) return fail(ctx, PRISM_HIP_ERR_SHAPE, "empty shape %ux%u", dm, dn);
  const size_t want = expected_bytes(dm, dn, bits);
  if (bytes != want)
    return fail(ctx, PRISM_HIP_ERR_SIZE, "payload is %zu bytes, %u-bit %ux%u needs %zu", bytes, bits, dm, dn, want);
  return PRISM_HIP_OK;
}

int ensure_stage(prism_hip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->stage_bytes) return PRISM_HIP_OK;
  if (ctx->d_stage) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipFree(ctx->d_stage));
    ctx->d_stage = nullptr;
    ctx->stage_bytes = 0;
  }
  size_t sz = 1 << 20;
  while (sz < bytes) sz <<= 1;
  HIP_TRY(ctx, hipMalloc(&ctx->d_stage, sz));
  ctx->stage_bytes = sz;
  return PRISM_HIP_OK;
}

int ensure_upload_stage(prism_hip_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->upload_bytes) return PRISM_HIP_OK;
  if (ctx->d_upload) {
    HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
    HIP_TRY(ctx, hipFree(ctx->d_upload));
    ctx->d_upload = nullptr;
    ctx->upload_bytes = 0;
  }
  size_t sz = 1 << 20;
  while (sz < bytes) sz <<= 1;
  HIP_TRY(ctx, hipMalloc(&ctx->d_upload, sz));
  ctx->upload_bytes = sz;
  return PRISM_HIP_OK;
}

// Host memcpy workers for the staging ring: copies of 512 KB and more are
// split into 256 KB parts that a few threads living for the whole process
// take in turn with the caller (one thread copies about 10-15 GB/s out of
// the page cache, the PCIe link takes several times that, and spawning
// threads per copy cost more than copying a 2 MB tensor).  One copy at a
// time; callers on several threads queue on `call_mu`.  The pool is never
// destroyed: its threads only ever run memcpy and end with the process.
class CopyPool {
 public:
  static CopyPool& get() {
    static CopyPool* p = new CopyPool();
    return *p;
  }
  void copy(void* dst, const void* src, size_t n) {
    constexpr size_t kPart = (size_t)256 << 10;
    if (n < 2 * kPart || workers_ == 0) {
      std::memcpy(dst, src, n);
      return;
    }
    std::lock_guard<std::mutex> call(call_mu_);
    {
      std::lock_guard<std::mutex> g(mu_);
      dst_ = static_cast<char*>(dst);
      src_ = static_cast<const char*>(src);
      n_ = n;
      finished_ = 0;
      total_ = (n + kPart - 1) / kPart;
      nparts_.store(total_);
      next_.store(0);
      gen_++;
    }
    cv_.notify_all();
    const size_t mine = work(kPart);
    std::unique_lock<std::mutex> g(mu_);
    finished_ += mine;
    // every part copied and every worker that took this job out of work()
    // (one still in it could otherwise claim a part of the next job)
    done_cv_.wait(g, [&] { return finished_ == total_ && active_ == 0; });
    nparts_.store(0);  // workers that wake late find no parts
  }

 private:
  CopyPool() {
    const unsigned hw = std::thread::hardware_concurrency();
    workers_ = std::min(7u, hw > 2 ? hw / 2 - 1 : 0u);
    for (unsigned i = 0; i < workers_; i++) std::thread([this] { loop(); }).detach();
  }
  // parts taken by this thread; the caller holds no lock
  size_t work(size_t part) {
    size_t done = 0;
    for (size_t i; (i = next_.fetch_add(1)) < nparts_.load();) {
      const size_t o = i * part, len = std::min(part, n_ - o);
      std::memcpy(dst_ + o, src_ + o, len);
      done++;
    }
    return done;
  }
  void loop() {
    uint64_t seen = 0;
    for (;;) {
      size_t part_bytes;
      {
        std::unique_lock<std::mutex> g(mu_);
        cv_.wait(g, [&] { return gen_ != seen; });
        seen = gen_;
        if (nparts_.load() == 0) continue;
        part_bytes = (size_t)256 << 10;
        active_++;
      }
      const size_t mine = work(part_bytes);
      std::lock_guard<std::mutex> g(mu_);
      finished_ += mine;
      active_--;
      if (finished_ == total_ && active_ == 0) done_cv_.notify_one();
    }
  }
  unsigned workers_ = 0;
  std::mutex call_mu_, mu_;
  std::condition_variable cv_, done_cv_;
  char* dst_ = nullptr;
  const char* src_ = nullptr;
  size_t n_ = 0, total_ = 0, finished_ = 0;
  unsigned active_ = 0;  // workers inside work() for the current job
  std::atomic<size_t> nparts_{0}, next_{0};
  uint64_t gen_ = 0;
};

void host_copy(void* dst, const void* src, size_t n) { CopyPool::get().copy(dst, src, n); }

// Host -> device copy of `bytes` through the pinned ring, in pieces of one
// slot: each piece waits for the last copy out of its slot, is copied into
// it on the host, and its device copy is enqueued on the context stream.
// `src` is consumed before the call returns; the device copies complete in
// stream order.
int stage_h2d(prism_hip_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx->ring[0]) {
    for (int i = 0; i < prism_hip_ctx::kRingSlots; i++) {
      HIP_TRY(ctx, hipHostMalloc(&ctx->ring[i], prism_hip_ctx::kRingSlotBytes, hipHostMallocDefault));
      HIP_TRY(ctx, hipEventCreateWithFlags(&ctx->ring_done[i], hipEventDisableTiming));
    }
  }
  for (size_t off = 0; off < bytes; off += prism_hip_ctx::kRingSlotBytes) {
    const size_t n = std::min(prism_hip_ctx::kRingSlotBytes, bytes - off);
    const int slot = ctx->ring_next;
    ctx->ring_next = (slot + 1) % prism_hip_ctx::kRingSlots;
    HIP_TRY(ctx, hipEventSynchronize(ctx->ring_done[slot]));
    host_copy(ctx->ring[slot], static_cast<const char*>(src) + off, n);
    HIP_TRY(ctx, hipMemcpyAsync(static_cast<char*>(dst) + off, ctx->ring[slot], n, hipMemcpyHostToDevice, ctx->stream));
    HIP_TRY(ctx, hipEventRecord(ctx->ring_done[slot], ctx->stream));
  }
  return PRISM_HIP_OK;
}

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// Drop one reference; the last one frees the chunk (hipFree waits for work
// still using it).
void chunk_release(WeightChunk* c) {
  if (!c || c->refs.fetch_sub(1) != 1) return;
  DeviceGuard g(c->device);
  (void)hipFree(c->base);
  delete c;
}

// `bytes` of device memory for a weight: *chunk gets a reference on the
// chunk it lies in.
int weight_alloc(prism_hip_ctx* ctx, size_t bytes, uint8_t** d, WeightChunk** chunk) {
  constexpr size_t kAlign = 256, kOwn = (size_t)16 << 20, kMaxChunk = (size_t)64 << 20;
  const size_t need = (bytes + kAlign - 1) / kAlign * kAlign;
  auto fresh = [&](size_t size, WeightChunk** out) -> int {
    auto* c = new WeightChunk;
    c->size = size;
    c->device = ctx->device;
    const hipError_t e = hipMalloc(&c->base, size);
    if (e != hipSuccess) {
      delete c;
      return fail(ctx, PRISM_HIP_ERR_DEVICE, "weight memory (%zu bytes): hipMalloc: %s", size, hipGetErrorString(e));
    }
    *out = c;
    return PRISM_HIP_OK;
  };
  if (need > kOwn) {
    WeightChunk* c = nullptr;
    const int rc = fresh(need, &c);
    if (rc) return rc;
    c->used = need;
    c->refs = 1;
    *d = c->base;
    *chunk = c;
    return PRISM_HIP_OK;
  }
  if (!ctx->carve || ctx->carve->used + need > ctx->carve->size) {
    // at least `need`: a weight of up to kOwn bytes may exceed the next size
    WeightChunk* c = nullptr;
    const int rc = fresh(std::max(ctx->next_chunk, need), &c);
    if (rc) return rc;
    c->refs = 1;  // the context's
    chunk_release(ctx->carve);
    ctx->carve = c;
    ctx->next_chunk = std::min(kMaxChunk, ctx->next_chunk * 2);
  }
  WeightChunk* c = ctx->carve;
  *d = c->base + c->used;
  c->used += need;
  c->refs.fetch_add(1);
  *chunk = c;
  return PRISM_HIP_OK;
}

int ensure_pool(prism_hip_ctx* ctx) {
  if (ctx->pool) return PRISM_HIP_OK;
  hipMemPoolProps props;
  std::memset(&props, 0, sizeof props);
  props.allocType = hipMemAllocationTypePinned;
  props.handleTypes = hipMemHandleTypeNone;
  props.location.type = hipMemLocationTypeDevice;
  props.location.id = ctx->device;
  hipMemPool_t pool = nullptr;
  HIP_TRY(ctx, hipMemPoolCreate(&pool, &props));
  uint64_t keep = UINT64_MAX;  // never trim at synchronisation points
  const hipError_t e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
  if (e != hipSuccess) {
    (void)hipMemPoolDestroy(pool);
    return fail(ctx, PRISM_HIP_ERR_DEVICE, "hipMemPoolSetAttribute: %s", hipGetErrorString(e));
  }
  ctx->pool = pool;
  return PRISM_HIP_OK;
}

int check_weight(prism_hip_ctx* ctx, const prism_hip_weight* w) {
  if (!w) return fail(ctx, PRISM_HIP_ERR_NULL, "weight is NULL");
  if (w->ctx != ctx) return fail(ctx, PRISM_HIP_ERR_CONTEXT, "weight was uploaded through another context");
  return PRISM_HIP_OK;
}

hipStream_t pick_stream(prism_hip_ctx* ctx, void* stream) {
  return stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
}

// GI device layout (gemv_lpr.hpp) for 4-bit matrices with rows of at least
// 2048 elements whose rows fill every CU in one round of groups of 32..64
// rows (one group per workgroup; the gate/up form holds two 64 KB table
// sets, one workgroup per CU): G = ceil(N / num_cu) rounded up to a
// multiple of 8, so N = 14336 takes 56-row groups on 256 CUs.  Returns G, or
// 0 for split-block.  MI355X, against k_gemv_tile on split-block weights:
// 14336 x 4096 6.7 (64-row groups, 224 of them) against 8.4 us, gate + up
// 2 x 14336 x 4096 12.3 us; 4864 x 896 3.5 against 3.05 us and 896 x 4864
// 6.3 against 3.2 us (too few rows).
// 4-bit matrices with more than 64 rows per CU, up to 128 (N <= 32768 on 256
// CUs), take 32-row groups and the half-group kernels (gemv_lpr.hpp, HG): a
// workgroup's 64 lanes hold two 32-row groups, two workgroups per CU.
// MI355X, 2 x 18944 x 3584 gate + up (592 workgroups of 32 + 32 rows):
// 13.8 us against 16.2-17.1 on split-block weights and 18.8 with 64-row
// groups (one gate + up workgroup per CU: 296 of them, two rounds); the
// one-matrix 18944 x 3584 GEMV 8.7 against 9.4 us.
// 8-bit matrices take the same groups when K % 512 == 0 (k_gemv_lpr8's
// eight waves split a row into whole blocks of four 16-byte chunks):
// 14336 x 4096 at 1 / 2 / 4 / 8 vectors 11.8 / 12.1 / 13.6 / 18.2 us
// against 14.3 / 15.5 / 18.2 / 19.8 on split-block weights; more than 64
// rows per CU stay split-block.
uint32_t gi_rows(const prism_hip_ctx* ctx, uint32_t dm, uint32_t dn, uint32_t bits) {
  if (dn < 2048 || (bits == 4 && dn % 64 != 0) || (bits == 8 && dn % 512 != 0) || (bits != 4 && bits != 8))
    return 0;
  const uint32_t ncu = (uint32_t)ctx->num_cu;
  uint32_t G = ((dm + ncu - 1) / ncu + 7) / 8 * 8;
  if (bits == 4 && G > (uint32_t)prism::kGiMaxRows && (dm + 63) / 64 <= 2 * ncu) G = 32;
  if (G < 32 || G > (uint32_t)prism::kGiMaxRows || prism::gi_bytes(G, dm, dn, bits) >= (1ull << 31)) return 0;
  return G;
}

// 4-bit GI weights run by the half-group kernels: 32-row groups, more of
// them than CUs (the 32-row groups of N <= 8192 run one group per
// workgroup, lanes 32..63 idle, so that every CU has one).
bool gi_half_groups(const prism_hip_ctx* ctx, const prism_hip_weight* w) {
  return w->bits == 4 && w->gi == 32 && (w->dim_m + 31) / 32 > (uint32_t)ctx->num_cu;
}

// ---------------------------------------------------------------- GEMV plan
// k_gemv_tile (gemv_tile.hpp) for K % 8 == 0 with 16-byte aligned x, in
// passes of up to 8 batch vectors (the matrix-core kernel of gemv_mfma.hpp
// takes several vectors over many rows, up to 16 a pass); k_gemv_generic
// otherwise.

struct TilePlan {
  const void* fn = nullptr;
  int threads = 0;
  int R = 1;
  size_t lds = 0;
};

// WI > 1: WI independent one-wave tiles per workgroup (threads == 64).
template <int BITS, int UPL, int R, bool DUAL, int NB, int EPI, int WI>
TilePlan tile_entry(int threads) {
  TilePlan p;
  p.fn = reinterpret_cast<const void*>(&prism::k_gemv_tile<BITS, UPL, R, DUAL, NB, EPI, WI>);
  if constexpr (WI > 1) {
    p.threads = 64 * WI;
    p.R = R * WI;
    p.lds = WI * prism::gemv_tile_wave_lds_bytes<BITS, R, DUAL, NB>();
  } else {
    p.threads = threads;
    p.R = R;
    p.lds = prism::gemv_tile_lds_bytes<BITS, R, DUAL, NB>(threads);
  }
  return p;
}

// Units per thread of the attention-combine prologue (kEpiAttnIn): at 6..8
// the unrolled combines spilled 8..148 VGPRs, so longer rows take more waves.
constexpr int kAttnInUplMax = 4;

// x units held in VGPRs: NB * UPL * 4 registers, at most 64.
template <int BITS, int R, bool DUAL, int NB, int EPI = 0, int WI = 1>
TilePlan tile_pick_upl(int upl, int threads) {
  switch (upl) {
#define PRISM_TU(u) \
  case u:           \
    if constexpr (NB * (u) <= 16 && ((EPI & prism::kEpiAttnIn) == 0 || (u) <= kAttnInUplMax)) \
      return tile_entry<BITS, u, R, DUAL, NB, EPI, WI>(threads);                                  \
    else                                                                                             \
      return TilePlan{};
    PRISM_TU(1) PRISM_TU(2) PRISM_TU(3) PRISM_TU(4) PRISM_TU(5) PRISM_TU(6) PRISM_TU(7) PRISM_TU(8)
#undef PRISM_TU
  }
  return TilePlan{};
}

// Rows per workgroup: 2 (4 tables for gate+up), 4 for 4+ batch vectors and
// for 8-bit weights (whose LUT loads are spread over >= 256 threads).
// `epi` (prism::kEpiNorm, kEpiResid, kEpiAttnIn | kEpiResid; decode step
// only) is 4-bit, batch 1.
TilePlan plan_tile(uint32_t bits, uint32_t N, uint32_t K, uint32_t nb, bool dual, uintptr_t xaddr, int epi = 0) {
  if (K % 8 != 0 || K == 0 || xaddr % 16 != 0) return TilePlan{};
  // buffer descriptors address the index block and x with 32-bit ranges
  if ((uint64_t)N * K * bits / 8 >= (1ull << 31) || (uint64_t)K * 2 >= (1ull << 31)) return TilePlan{};
  const uint32_t U = K / 8;
  const int NB = nb <= 1 ? 1 : nb <= 2 ? 2 : nb <= 4 ? 4 : 8;
  if (dual && NB != 1) return TilePlan{};
  if (epi == prism::kEpiPair ? !dual : epi && (NB != 1 || bits != 4)) return TilePlan{};
  const uint32_t uplmax = (epi & prism::kEpiAttnIn) ? (uint32_t)kAttnInUplMax : (uint32_t)(16 / NB < 8 ? 16 / NB : 8);
  // Very tall single-vector 4-bit matrices (an LM head: N >= 32768) take 4
  // rows per wave: at 2 rows, dispatching N/2 workgroups costs more than
  // their bytes (measured on 151936 x 896: 47 us at R=2, 26 us at R=4), and
  // one-wave tiles go four to a workgroup (below).
  const bool tall = bits == 4 && NB == 1 && !dual && N >= 32768;
  // 4-bit single-vector rows of 65..128 units (K <= 1024, the decode step's
  // and cfg1's shapes): two independent one-wave tiles per workgroup.
  // MI355X: 4864x896 3.04 against 3.22 us with one two-wave tile (K split
  // over the waves), the Qwen2.5-0.5B decode step 540 against 553 us/token;
  // four tiles: 3.06 / 543.  Longer rows (cfg2's gate_up, K = 3584) lost
  // with two or four (17.2 against 16.4 us).
  const bool pair = bits == 4 && NB == 1 && !tall && U > 64 && U <= 128;
  // waves per workgroup: the fewest that keep UPL <= uplmax; 8-bit rows at
  // least 4
  uint32_t W = 0;
  const uint32_t wmin = bits == 8 ? 4u : 1u;
  for (uint32_t w = wmin; w <= 8; w *= 2)
    if ((U + 64 * w - 1) / (64 * w) <= uplmax) {
      W = w;
      break;
    }
  if (!W) return TilePlan{};
  const int upl = (int)((U + 64 * W - 1) / (64 * W));
  const int threads = (int)(64 * W);
  if (bits == 4) {
    if (pair) {
      if (dual) {
        if (epi == prism::kEpiNorm) return tile_pick_upl<4, 2, true, 1, prism::kEpiNorm, 2>(upl, threads);
        if (epi == prism::kEpiPair) return tile_pick_upl<4, 2, true, 1, prism::kEpiPair, 2>(upl, threads);
        if (epi) return TilePlan{};
        return tile_pick_upl<4, 2, true, 1, 0, 2>(upl, threads);
      }
      if (epi == prism::kEpiNorm) return tile_pick_upl<4, 2, false, 1, prism::kEpiNorm, 2>(upl, threads);
      if (epi == prism::kEpiResid) return tile_pick_upl<4, 2, false, 1, prism::kEpiResid, 2>(upl, threads);
      if (epi == (prism::kEpiAttnIn | prism::kEpiResid))
        return tile_pick_upl<4, 2, false, 1, prism::kEpiAttnIn | prism::kEpiResid, 2>(upl, threads);
      if (epi) return TilePlan{};
      return tile_pick_upl<4, 2, false, 1, 0, 2>(upl, threads);
    }
    if (dual) {
      if (epi == prism::kEpiNorm) return tile_pick_upl<4, 2, true, 1, prism::kEpiNorm>(upl, threads);
      if (epi == prism::kEpiPair) return tile_pick_upl<4, 2, true, 1, prism::kEpiPair>(upl, threads);
      if (epi) return TilePlan{};
      return tile_pick_upl<4, 2, true, 1>(upl, threads);
    }
    if (tall) {
      // one-wave tiles, four to a workgroup: 151936 x 896 in 20.0 us against
      // 24.8 with one tile per workgroup (38 K workgroups to dispatch)
      if (W == 1) {
        if (epi == prism::kEpiNorm) return tile_pick_upl<4, 4, false, 1, prism::kEpiNorm, 4>(upl, threads);
        if (epi == prism::kEpiResid) return tile_pick_upl<4, 4, false, 1, prism::kEpiResid, 4>(upl, threads);
        if (epi) return TilePlan{};
        return tile_pick_upl<4, 4, false, 1, 0, 4>(upl, threads);
      }
      if (epi == prism::kEpiNorm) return tile_pick_upl<4, 4, false, 1, prism::kEpiNorm>(upl, threads);
      if (epi == prism::kEpiResid) return tile_pick_upl<4, 4, false, 1, prism::kEpiResid>(upl, threads);
      if (epi) return TilePlan{};
      return tile_pick_upl<4, 4, false, 1>(upl, threads);
    }
    if (epi == prism::kEpiNorm) return tile_pick_upl<4, 2, false, 1, prism::kEpiNorm>(upl, threads);
    if (epi == prism::kEpiResid) return tile_pick_upl<4, 2, false, 1, prism::kEpiResid>(upl, threads);
    if (epi == (prism::kEpiAttnIn | prism::kEpiResid))
      return tile_pick_upl<4, 2, false, 1, prism::kEpiAttnIn | prism::kEpiResid>(upl, threads);
    if (epi) return TilePlan{};
    switch (NB) {
      case 1: return tile_pick_upl<4, 2, false, 1>(upl, threads);
      case 2: return tile_pick_upl<4, 2, false, 2>(upl, threads);
      case 4: return tile_pick_upl<4, 4, false, 4>(upl, threads);
      default: return tile_pick_upl<4, 4, false, 8>(upl, threads);
    }
  }
  if (dual) {
    if (epi == prism::kEpiPair) return tile_pick_upl<8, 2, true, 1, prism::kEpiPair>(upl, threads);
    return tile_pick_upl<8, 2, true, 1>(upl, threads);
  }
  switch (NB) {
    case 1: return tile_pick_upl<8, 4, false, 1>(upl, threads);
    case 2: return tile_pick_upl<8, 4, false, 2>(upl, threads);
    case 4: return tile_pick_upl<8, 4, false, 4>(upl, threads);
    default: return tile_pick_upl<8, 4, false, 8>(upl, threads);
  }
}

// GEMV over raw split-block device pointers (lut2/idx2 non-null: gate+up
// with the SwiGLU epilogue, or with d_y2 non-null the two raw outputs).
// `epi` selects the decode step's fused norm / residual forms, which have no
// generic fallback.
int launch_gemv_raw(prism_hip_ctx* ctx, uint32_t bits, uint32_t N, uint32_t K, const uint8_t* lut,
                    const uint8_t* idx, const uint8_t* lut2, const uint8_t* idx2, const void* d_x, uint32_t nb,
                    void* d_y, hipStream_t st, int epi = 0, float eps = 0.0f, const float* xpart = nullptr,
                    void* d_y2 = nullptr) {
  const bool dual = (lut2 != nullptr);
  const bool pair = dual && d_y2 != nullptr;
  if (pair) epi = prism::kEpiPair;
  prism::GemvArgs a;
  a.lut = lut;
  a.idx = idx;
  a.lut2 = lut2;
  a.idx2 = idx2;
  a.y2 = reinterpret_cast<uint16_t*>(d_y2);
  a.N = N;
  a.K = K;
  a.eps = eps;
  a.xpart = xpart;
  for (uint32_t b0 = 0; b0 < nb;) {
    uint32_t chunk = (nb - b0 < 8) ? nb - b0 : 8;
    const uint32_t wide = (nb - b0 < (uint32_t)prism::kGmMaxNb) ? nb - b0 : (uint32_t)prism::kGmMaxNb;
    a.x = reinterpret_cast<const uint16_t*>(d_x) + (size_t)b0 * K;
    a.y = reinterpret_cast<uint16_t*>(d_y) + (size_t)b0 * N;
    void* args[] = {&a};
    // Several batch vectors over 4096 rows or more: the matrix-core kernel
    // (gemv_mfma.hpp), from 5 vectors, and for 4-bit rows up to 8192 long
    // from 3 (from 2 over 8192 rows or more).  Against the tile kernel on
    // MI355X: 4-bit 14336x4096 at 8 / 4 / 3 / 2 vectors 11.2 / 10.0 / 9.9 /
    // 9.6 vs 21.8 / 13.3 / 12.9 / 10.2 us; 8-bit at 8 vectors 19.6 vs 26.0
    // us, 29.8 vs 2 x 20 at 4096x14336, 6.1 vs 7.8 at 4864x896.  Slower with
    // fewer rows (2048: 64 workgroups), at one vector (9.5 vs 8.6), for 4-bit
    // at 2 vectors over 4864 rows (4.1 vs 3.6), for 8-bit at 3..4 vectors and
    // for long 4-bit rows at 3..4 (4096x14336: 16.5 vs 14.8).
    // It takes up to 16 vectors a pass, the tile kernel 8.
    const bool mfma_batch =
        wide >= 5 || (bits == 4 && K <= 8192 && (wide >= 3 || (wide == 2 && N >= 8192)));
    if (!dual && !epi && mfma_batch && N >= 4096 && K % prism::kGmGroup == 0 &&
        (uint64_t)N * K * bits / 8 < (1ull << 31) && reinterpret_cast<uintptr_t>(a.x) % 16 == 0) {
      chunk = wide;
      a.nb = chunk;
      const void* fn = bits == 8 ? reinterpret_cast<const void*>(&prism::k_gemv_mfma<8>)
                                 : reinterpret_cast<const void*>(&prism::k_gemv_mfma<4>);
      HIP_TRY(ctx, launch_fn(fn, dim3((N + prism::kGmRows - 1) / prism::kGmRows), dim3(64 * prism::kGmWaves),
                                   args, 0, st));
      b0 += chunk;
      continue;
    }
    TilePlan p = plan_tile(bits, N, K, chunk, dual, reinterpret_cast<uintptr_t>(a.x), epi);
    // rows too long for the tile kernel's registers at this many vectors:
    // fewer vectors per pass (each pass streams the weights again, still far
    // cheaper than the generic kernel: 2 x 20 us against 830 us for 8
    // vectors on 4096x14336 8-bit)
    for (uint32_t c = chunk; !p.fn && c > 1 && !epi && !dual;) {
      c = c > 4 ? 4 : c > 2 ? 2 : 1;
      const TilePlan q = plan_tile(bits, N, K, c, dual, reinterpret_cast<uintptr_t>(a.x), epi);
      if (q.fn) {
        p = q;
        chunk = c;
      }
    }
    a.nb = chunk;
    if (p.fn) {
      const uint32_t grid = (N + (uint32_t)p.R - 1) / (uint32_t)p.R;
      HIP_TRY(ctx, launch_fn(p.fn, dim3(grid), dim3(p.threads), args, p.lds, st));
    } else {
      if (epi && !pair) return fail(ctx, PRISM_HIP_ERR_SHAPE, "no fused kernel for %u-bit %ux%u", bits, N, K);
      const void* fn;
      if (pair)
        fn = bits == 4 ? reinterpret_cast<const void*>(&prism::k_gemv_generic<4, prism::kGenPair>)
                       : reinterpret_cast<const void*>(&prism::k_gemv_generic<8, prism::kGenPair>);
      else if (dual)
        fn = bits == 4 ? reinterpret_cast<const void*>(&prism::k_gemv_generic<4, prism::kGenSwiglu>)
                       : reinterpret_cast<const void*>(&prism::k_gemv_generic<8, prism::kGenSwiglu>);
      else
        fn = bits == 4 ? reinterpret_cast<const void*>(&prism::k_gemv_generic<4, prism::kGenSingle>)
                       : reinterpret_cast<const void*>(&prism::k_gemv_generic<8, prism::kGenSingle>);
      HIP_TRY(ctx, launch_fn(fn, dim3(N), dim3(64), args, 0, st));
    }
    b0 += chunk;
  }
  return PRISM_HIP_OK;
}

// GEMV over GI weights (w2: gate + up, SwiGLU or with d_y2 the pair).
// One or two vectors a pass: k_gemv_lpr; three to eight over groups of more
// than 32 rows, K % 256 == 0 and x within its LDS: k_gemv_lpr4m; otherwise
// three or more: the matrix-core kernel (K % 128 == 0) in passes of up to
// 16, else lane-per-row passes of two.  x not 16-byte aligned: the generic
// kernel.
// k_gemv_lpr with the wave's chunk count as a compile-time constant when
// every wave has the same count (K/32 a multiple of S) and it is 8 or 16,
// else the run-time loop.
template <int S, int NM, int NB, int EPI>
void launch_lpr(dim3 groups, hipStream_t st, const prism::LprArgs& a) {
  const uint32_t NC = a.K / 32;
  const uint32_t nch = NC % S == 0 ? NC / S : 0;
  if (nch == 16)
    PRISM_LAUNCH((prism::k_gemv_lpr<S, NM, NB, EPI, 16>), groups, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if (nch == 8)
    PRISM_LAUNCH((prism::k_gemv_lpr<S, NM, NB, EPI, 8>), groups, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else
    PRISM_LAUNCH((prism::k_gemv_lpr<S, NM, NB, EPI>), groups, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
}

// The half-group form (G = 32), with a compile-time chunk count as above,
// and also for 14 chunks per wave (K = 3584 at 8 waves, config 2's rows:
// gate + up 13.8 against 14.55 us for the run-time loop, MI355X; 16 waves
// 16.6, and 15.3-15.4 with 7 compile-time chunks each).
template <int S, int NM, int NB, int EPI>
void launch_lpr_hg(dim3 grid, hipStream_t st, const prism::LprArgs& a) {
  const uint32_t NC = a.K / 32;
  const uint32_t nch = NC % S == 0 ? NC / S : 0;
  if (nch == 16)
    PRISM_LAUNCH((prism::k_gemv_lpr_hg<S, NM, NB, EPI, 16>), grid, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if (nch == 14)
    PRISM_LAUNCH((prism::k_gemv_lpr_hg<S, NM, NB, EPI, 14>), grid, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if (nch == 8)
    PRISM_LAUNCH((prism::k_gemv_lpr_hg<S, NM, NB, EPI, 8>), grid, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else
    PRISM_LAUNCH((prism::k_gemv_lpr_hg<S, NM, NB, EPI>), grid, dim3(64 * S), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
}

// 8-bit GI weights: k_gemv_lpr8 with the wave's chunk count as a
// compile-time constant when it is 16, 32 or 64 (K = 2048 / 4096 / 8192),
// else the loop over 4-chunk blocks.  Eight vectors a pass only with a
// compile-time count (the loop form runs out of SGPRs for their x).
bool lpr8_static(uint32_t K) {
  const uint32_t nch = K / 16 / 8;
  return nch == 16 || nch == 32 || nch == 64;
}
// Eight vectors with a run-time chunk count have no kernel: that returns an
// error (the dispatch below never asks for it) instead of launching nothing.
template <int NM, int NB, int EPI>
int launch_lpr8(prism_hip_ctx* ctx, dim3 groups, hipStream_t st, const prism::LprArgs& a) {
  const uint32_t nch = a.K / 16 / 8;
  if (nch == 32)
    PRISM_LAUNCH((prism::k_gemv_lpr8<8, NM, NB, EPI, 32>), groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if (nch == 16)
    PRISM_LAUNCH((prism::k_gemv_lpr8<8, NM, NB, EPI, 16>), groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if (nch == 64)
    PRISM_LAUNCH((prism::k_gemv_lpr8<8, NM, NB, EPI, 64>), groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else if constexpr (NB < 8)
    PRISM_LAUNCH((prism::k_gemv_lpr8<8, NM, NB, EPI>), groups, dim3(512), 0, st, a.w, a.w2, a.x, a.y, a.y2, a.N, a.K, a.nb, a.G);
  else
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "k_gemv_lpr8: %d vectors need a compile-time chunk count (K = %u)", NB,
                a.K);
  return PRISM_HIP_OK;
}

// GEMV over 8-bit GI weights: gate + up (SwiGLU, or the pair with d_y2) in
// one k_gemv_lpr8 pass; one matrix in passes of 1 / 2 vectors (k_gemv_lpr8),
// of 3..8 with the lane-per-row lookups feeding the matrix cores when x fits
// their LDS (k_gemv_lpr8m: nb * (K / 2 + 4) <= 16512), else of 4 or 8
// (k_gemv_lpr8; 3..4 vectors then have K > 8248, so the run-time chunk loop),
// or of up to 16 on the matrix cores from 9 vectors on (from 5 when the
// chunk count is not a compile-time one and x does not fit k_gemv_lpr8m)
// (k_gemv_mfma<8, GI>).  x not 16-byte aligned: the generic kernel.
// Config 4 (14336 x 4096), MI355X, alternating on one box: 3 / 4 vectors
// 12.77-12.81 / 12.95-13.05 us on k_gemv_lpr8m against 13.37-13.50 /
// 13.27-13.39 on k_gemv_lpr8; 2 vectors 12.73-12.80 against 11.92-11.96, so
// 2 stay with k_gemv_lpr8.
int launch_gemv_gi8(prism_hip_ctx* ctx, const prism_hip_weight* w, const prism_hip_weight* w2, const void* d_x,
                    uint32_t nb, void* d_y, void* d_y2, hipStream_t st) {
  const uint32_t N = w->dim_m, K = w->dim_n;
  const bool aligned = reinterpret_cast<uintptr_t>(d_x) % 16 == 0;
  const uint32_t G = w->gi;
  const dim3 groups((N + G - 1) / G);
  prism::GemvArgs ga{};
  ga.gi = G;
  ga.lut = ga.idx = w->d;
  ga.N = N;
  ga.K = K;
  if (w2) {
    ga.lut2 = ga.idx2 = w2->d;
    ga.x = reinterpret_cast<const uint16_t*>(d_x);
    ga.y = reinterpret_cast<uint16_t*>(d_y);
    ga.y2 = reinterpret_cast<uint16_t*>(d_y2);
    ga.nb = 1;
    if (aligned) {
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.w2 = w2->d;
      a.x = ga.x;
      a.y = ga.y;
      a.y2 = ga.y2;
      a.N = N;
      a.K = K;
      a.nb = 1;
      const int rc = d_y2 ? launch_lpr8<2, 1, prism::kLprPair>(ctx, groups, st, a)
                          : launch_lpr8<2, 1, prism::kLprSwiglu>(ctx, groups, st, a);
      if (rc) return rc;
    } else if (d_y2) {
      PRISM_LAUNCH((prism::k_gemv_generic<8, prism::kGenPair, true>), dim3(N), dim3(64), 0, st, ga);
    } else {
      PRISM_LAUNCH((prism::k_gemv_generic<8, prism::kGenSwiglu, true>), dim3(N), dim3(64), 0, st, ga);
    }
    HIP_TRY(ctx, hipGetLastError());
    return PRISM_HIP_OK;
  }
  for (uint32_t b0 = 0; b0 < nb;) {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(d_x) + (size_t)b0 * K;
    uint16_t* y = reinterpret_cast<uint16_t*>(d_y) + (size_t)b0 * N;
    const uint32_t left = nb - b0;
    uint32_t chunk;
    if (!aligned) {
      ga.x = x;
      ga.y = y;
      ga.nb = chunk = left;
      PRISM_LAUNCH((prism::k_gemv_generic<8, prism::kGenSingle, true>), dim3(N), dim3(64), 0, st, ga);
    } else if (left >= 3 && left <= 8 && left * (K / 2 + prism::kLpr8mXPad) <= (uint32_t)prism::kLpr8mXDw) {
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left;
      HIP_TRY(ctx, prism::launch_gemv_lpr8m(groups, st, a));
    } else if (left >= 9 || (left >= 5 && !lpr8_static(K))) {
      ga.x = x;
      ga.y = y;
      ga.nb = chunk = left < (uint32_t)prism::kGmMaxNb ? left : (uint32_t)prism::kGmMaxNb;
      PRISM_LAUNCH((prism::k_gemv_mfma<8, true>), dim3((N + prism::kGmRows - 1) / prism::kGmRows),
                   dim3(64 * prism::kGmWaves), 0, st, ga);
    } else {
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left;
      const int rc = left == 1   ? launch_lpr8<1, 1, prism::kLprPlain>(ctx, groups, st, a)
                     : left == 2 ? launch_lpr8<1, 2, prism::kLprPlain>(ctx, groups, st, a)
                     : left <= 4 ? launch_lpr8<1, 4, prism::kLprPlain>(ctx, groups, st, a)
                                 : launch_lpr8<1, 8, prism::kLprPlain>(ctx, groups, st, a);
      if (rc) return rc;
    }
    HIP_TRY(ctx, hipGetLastError());
    b0 += chunk;
  }
  return PRISM_HIP_OK;
}

int launch_gemv_gi(prism_hip_ctx* ctx, const prism_hip_weight* w, const prism_hip_weight* w2, const void* d_x,
                   uint32_t nb, void* d_y, void* d_y2, hipStream_t st) {
  if (w->bits == 8) return launch_gemv_gi8(ctx, w, w2, d_x, nb, d_y, d_y2, st);
  const uint32_t N = w->dim_m, K = w->dim_n;
  const bool aligned = reinterpret_cast<uintptr_t>(d_x) % 16 == 0;
  const uint32_t G = w->gi;
  const dim3 groups((N + G - 1) / G);
  const bool hg = gi_half_groups(ctx, w);
  if (w2) {
    if (aligned) {
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.w2 = w2->d;
      a.x = reinterpret_cast<const uint16_t*>(d_x);
      a.y = reinterpret_cast<uint16_t*>(d_y);
      a.y2 = reinterpret_cast<uint16_t*>(d_y2);
      a.N = N;
      a.K = K;
      a.nb = 1;
      // the pair form splits K over the waves as the one-matrix GEMV does
      // (8 waves), so each output is that GEMV's bit for bit
      if (hg) {
        if (d_y2)
          launch_lpr_hg<8, 2, 1, prism::kLprPair>(groups, st, a);
        else
          launch_lpr_hg<8, 2, 1, prism::kLprSwiglu>(groups, st, a);
      } else if (d_y2)
        launch_lpr<8, 2, 1, prism::kLprPair>(groups, st, a);
      else
        launch_lpr<16, 2, 1, prism::kLprSwiglu>(groups, st, a);
    } else {
      prism::GemvArgs a{};
      a.gi = G;
      a.lut = a.idx = w->d;
      a.lut2 = a.idx2 = w2->d;
      a.x = reinterpret_cast<const uint16_t*>(d_x);
      a.y = reinterpret_cast<uint16_t*>(d_y);
      a.y2 = reinterpret_cast<uint16_t*>(d_y2);
      a.N = N;
      a.K = K;
      a.nb = 1;
      if (d_y2)
        PRISM_LAUNCH((prism::k_gemv_generic<4, prism::kGenPair, true>), dim3(N), dim3(64), 0, st, a);
      else
        PRISM_LAUNCH((prism::k_gemv_generic<4, prism::kGenSwiglu, true>), dim3(N), dim3(64), 0, st, a);
    }
    HIP_TRY(ctx, hipGetLastError());
    return PRISM_HIP_OK;
  }
  for (uint32_t b0 = 0; b0 < nb;) {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(d_x) + (size_t)b0 * K;
    uint16_t* y = reinterpret_cast<uint16_t*>(d_y) + (size_t)b0 * N;
    const uint32_t left = nb - b0;
    uint32_t chunk;
    if (!aligned) {
      prism::GemvArgs a{};
      a.gi = G;
      a.lut = a.idx = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left;
      PRISM_LAUNCH((prism::k_gemv_generic<4, prism::kGenSingle, true>), dim3(N), dim3(64), 0, st, a);
    } else if (!hg && G > 32 && (left == 3 || left == 4) && K % 256 == 0 &&
               left * (K / 2 + prism::kLpr8mXPad) <= (uint32_t)prism::kLpr8mXDw) {
      // 3..4 vectors over groups of 33..64 rows: k_gemv_lpr4q, the lane-per-row
      // lookups feeding 4 x 4 x 4 matrix-core blocks.  MI355X, 14336 x 4096,
      // bench.py alternating on one box: 3 / 4 vectors 8.04-8.21 /
      // 8.10-8.25 us against 8.39-8.50 / 8.43-8.61 for k_gemv_lpr4m.
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left;
      HIP_TRY(ctx, prism::launch_gemv_lpr4q(groups, st, a));
    } else if (!hg && G > 32 && left >= 3 && left <= 8 && K % 256 == 0 &&
               left * (K / 2 + prism::kLpr8mXPad) <= (uint32_t)prism::kLpr8mXDw) {
      // 3..8 vectors over groups of 33..64 rows (both row tiles of
      // k_gemv_lpr4m busy) when x fits its LDS.  MI355X, 14336 x 4096,
      // alternating on one box: 3 / 4 / 8 vectors 8.16-8.24 / 8.26-8.29 /
      // 9.02 us against 9.40-9.42 / 9.48-9.51 / 10.07-10.22 for
      // k_gemv_mfma<4, GI>; 1 / 2 vectors 7.97 / 8.07-8.13 against
      // 6.36-6.38 / 7.59-7.91 for k_gemv_lpr, which keeps them.
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left;
      HIP_TRY(ctx, prism::launch_gemv_lpr4m(groups, st, a));
    } else if (left >= 3 && K % prism::kGmGroup == 0) {
      prism::GemvArgs a{};
      a.gi = G;
      a.lut = a.idx = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left < (uint32_t)prism::kGmMaxNb ? left : (uint32_t)prism::kGmMaxNb;
      PRISM_LAUNCH((prism::k_gemv_mfma<4, true>), dim3((N + prism::kGmRows - 1) / prism::kGmRows),
                   dim3(64 * prism::kGmWaves), 0, st, a);
    } else {
      prism::LprArgs a{};
      a.G = G;
      a.w = w->d;
      a.x = x;
      a.y = y;
      a.N = N;
      a.K = K;
      a.nb = chunk = left >= 2 ? 2u : 1u;
      if (hg) {
        const dim3 pairs((groups.x + 1) / 2);
        if (chunk == 2)
          launch_lpr_hg<8, 1, 2, prism::kLprPlain>(pairs, st, a);
        else
          launch_lpr_hg<8, 1, 1, prism::kLprPlain>(pairs, st, a);
      } else if (chunk == 2)
        launch_lpr<8, 1, 2, prism::kLprPlain>(groups, st, a);
      else
        launch_lpr<8, 1, 1, prism::kLprPlain>(groups, st, a);
    }
    HIP_TRY(ctx, hipGetLastError());
    b0 += chunk;
  }
  return PRISM_HIP_OK;
}

int launch_gemv(prism_hip_ctx* ctx, const prism_hip_weight* w, const prism_hip_weight* w2, const void* d_x,
                uint32_t nb, void* d_y, hipStream_t st, void* d_y2 = nullptr) {
  if (w->gi) return launch_gemv_gi(ctx, w, w2, d_x, nb, d_y, d_y2, st);
  return launch_gemv_raw(ctx, w->bits, w->dim_m, w->dim_n, w->lut(), w->idx(), w2 ? w2->lut() : nullptr,
                         w2 ? w2->idx() : nullptr, d_x, nb, d_y, st, 0, 0.0f, nullptr, d_y2);
}

// One GEMM kernel launch over (tiles, splits) blocks, kernel signature
// (lut, idx, X, Y, M, N, K, partials, K steps per split).  With nsplit > 1
// the K steps are cut into splits of kps steps (every split keeps at least
// one), the blocks write fp32 partials to a buffer from the context's
// stream-ordered pool, and k_gemm_split_sum adds them in split order.
// With `fixed` non-NULL the partials go there instead (at most
// kScratchBytes; nothing is allocated or freed).
int launch_gemm_blocks(prism_hip_ctx* ctx, const void* fn, uint32_t tiles, uint32_t nsteps, uint32_t nsplit,
                       const prism_hip_weight* w, const void* d_X, uint32_t M, void* d_Y, hipStream_t st,
                       float* fixed) {
  const uint8_t* lut = w->lut();
  const uint8_t* idx = w->idx();
  const uint16_t* X = reinterpret_cast<const uint16_t*>(d_X);
  uint16_t* Y = reinterpret_cast<uint16_t*>(d_Y);
  uint32_t N = w->dim_m, K = w->dim_n;
  const bool split = nsplit > 1;
  float* P = nullptr;
  uint32_t kps = 0, ns = 1;
  if (split) {
    kps = (nsteps + nsplit - 1) / nsplit;
    ns = (nsteps + kps - 1) / kps;
    const size_t pbytes = (size_t)ns * M * N * 4;
    if (fixed) {
      if (pbytes > kScratchBytes)
        return fail(ctx, PRISM_HIP_ERR_SIZE, "split-K partials of %zu bytes exceed the %zu-byte static scratch",
                    pbytes, kScratchBytes);
      P = fixed;
    } else {
      int rc = ensure_pool(ctx);
      if (rc) return rc;
      HIP_TRY(ctx, hipMallocFromPoolAsync(reinterpret_cast<void**>(&P), pbytes, ctx->pool, st));
    }
  }
  uint32_t G = w->gi;  // GI group rows (0: split-block; k_gemm8 ignores it)
  void* args[] = {&lut, &idx, &X, &Y, &M, &N, &K, &P, &kps, &G};
  hipError_t e = launch_fn(fn, dim3(tiles, ns), dim3(256), args, 0, st);
  if (e == hipSuccess && split) {
    const uint64_t mn = (uint64_t)M * N;
    PRISM_LAUNCH(prism::k_gemm_split_sum, dim3((unsigned)((mn + 1023) / 1024)), dim3(256), 0, st, P, Y, mn, ns);
    e = hipGetLastError();
  }
  if (split && !fixed) {
    const hipError_t f = hipFreeAsync(P, st);
    if (e == hipSuccess) e = f;
  }
  if (e != hipSuccess) return fail(ctx, PRISM_HIP_ERR_DEVICE, "GEMM launch: %s", hipGetErrorString(e));
  return PRISM_HIP_OK;
}

int launch_gemm(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_X, uint32_t M, void* d_Y,
                hipStream_t st, float* fixed = nullptr) {
  const uint32_t N = w->dim_m, K = w->dim_n, bits = w->bits;
  const bool fast = (K % prism::GEMM_BK == 0) && (reinterpret_cast<uintptr_t>(d_X) % 16 == 0);
  // Up to 32 rows of X (48 for 8-bit weights): GEMV passes of up to 16
  // vectors stream the weights M / 16 times but take less than the GEMM's
  // fixed cost.  MI355X, 14336x4096 4-bit: M = 24 / 32 / 40 / 48 take 25.7 /
  // 28.2 / 38.2 / 41.6 us as GEMVs and 31.1 / 31.5 / 31.9 / 32.8 us as the
  // split-K GEMM; 8-bit M = 32 / 48 / 64: 42.6 / 63.4 / 84.5 us against 65.2
  // / 65.4 / 66.2 us.
  if (!fast || M <= (bits == 8 ? 48u : 32u)) return launch_gemv(ctx, w, nullptr, d_X, M, d_Y, st);
  // 4-bit, K % 64 == 0: the MFMA kernel with register decode and LDS-DMA
  // staging (gemm_kernels.hpp, k_gemm_w4); its buffer descriptors address
  // the index block and one block's X rows with 32-bit ranges.  Blocks of
  // 32 * mi rows of X: short prefills take shorter blocks, so that more of
  // them fill the GPU.  MI355X, 14336x4096, mi = 2 / 4 / 8: M = 128 53.8 /
  // 67.8 / 106.2 us, M = 256 63.7 / 71.6 / 108.1, M = 512 110.3 / 89.8 /
  // 114.6, M = 640 - / 150.7 / 127.7, M = 2048 373.7 / 334.3 / 279.8.
  // Short 4-bit prefills split K: a block decodes its 256 weight rows over
  // its K range whatever its M rows, so up to 256 rows of X one M block of
  // 128 or 256 rows takes the whole GPU in K splits (at most 4, at least 8
  // K steps each; fp32 partials from the context's stream-ordered pool,
  // added in split order by k_gemm_split_sum).  MI355X, 14336x4096, M = 64 /
  // 128 / 192 / 256: 33.3 / 37.4 / 53.4 / 57.0 us against 52.6 / 54.6 / 58.9
  // / 65.6 unsplit; two splits, or 64-row blocks, came between; at 384 and
  // 512 rows splitting lost (88.7 / 94.1 against 79.9 / 89.6 us).
  const uint32_t nsteps = K / prism::GW4_BK;
  const uint32_t ntn = (N + prism::GW4_BN - 1) / prism::GW4_BN;
  uint32_t nsplit = 1;
  int mi = M <= 256 ? 2 : M <= 512 ? 4 : 8;
  if (M <= 256) {
    const int smi = M <= 128 ? 4 : 8;
    const uint32_t blocks = ((M + 32u * smi - 1) / (32u * smi)) * ntn;
    uint32_t sk = (uint32_t)ctx->num_cu / blocks;
    sk = sk < 4 ? sk : 4;
    sk = sk < nsteps / 8 ? sk : nsteps / 8;
    if (sk >= 2) {
      nsplit = sk;
      mi = smi;
    }
  }
  const uint32_t bm = 32u * (uint32_t)mi;
  if (bits == 4 && K % prism::GW4_BK == 0 && (uint64_t)N * (K / 2) < (1ull << 31) &&
      (uint64_t)bm * K * 2 < (1ull << 31)) {
    const uint32_t tiles4 = ((M + bm - 1) / bm) * ntn;
    const void* fn;
#define PRISM_W4(MI_, SP_)                                                                   \
  (w->gi ? reinterpret_cast<const void*>(&prism::k_gemm_w4<MI_, SP_, true>)                  \
           : reinterpret_cast<const void*>(&prism::k_gemm_w4<MI_, SP_, false>))
    if (nsplit > 1)
      fn = mi == 2 ? PRISM_W4(2, true) : mi == 4 ? PRISM_W4(4, true) : PRISM_W4(8, true);
    else
      fn = mi == 2 ? PRISM_W4(2, false) : mi == 4 ? PRISM_W4(4, false) : PRISM_W4(8, false);
#undef PRISM_W4
    return launch_gemm_blocks(ctx, fn, tiles4, nsteps, nsplit, w, d_X, M, d_Y, st, fixed);
  }
  // 8-bit, K % 64 == 0, more than 256 rows: 256 x 128 blocks over a 64-wide
  // K step (k_gemm8).  MI355X, 14336x4096: M = 384 / 512 / 2048 take 118 /
  // 123 / 454 us against 197 / 206 / 701 us in k_gemm<8>'s 128 x 128 blocks.
  // Up to 256 rows, one M block in K splits as for 4-bit (at most 4, at
  // least 8 K steps each; two at 14336 rows): M = 65 / 128 / 256 in 69.1 /
  // 72.5 / 77.0 us against 95.9 / 97.8 / 102.8 in k_gemm<8>, which is left
  // for prefills that cannot split.
  static_assert(prism::GM8_BK == prism::GW4_BK, "one K step for both GEMMs");
  if (bits == 8 && K % prism::GM8_BK == 0) {
    const uint32_t nt8 = (N + prism::GM8_BN - 1) / prism::GM8_BN;
    uint32_t sk8 = 1;
    if (M <= 256) {
      sk8 = (uint32_t)ctx->num_cu / nt8;
      sk8 = sk8 < 4 ? sk8 : 4;
      sk8 = sk8 < nsteps / 8 ? sk8 : nsteps / 8;
    }
    // GI weights always take k_gemm8 (unsplit when K cannot split)
    if (M > 256 || sk8 >= 2 || w->gi) {
      const uint32_t tiles8 = ((M + prism::GM8_BM - 1) / prism::GM8_BM) * nt8;
      const uint32_t nsplit8 = M <= 256 && sk8 >= 2 ? sk8 : 1;
      const void* fn = w->gi ? (nsplit8 > 1 ? reinterpret_cast<const void*>(&prism::k_gemm8<true, true>)
                                            : reinterpret_cast<const void*>(&prism::k_gemm8<false, true>))
                             : (nsplit8 > 1 ? reinterpret_cast<const void*>(&prism::k_gemm8<true>)
                                            : reinterpret_cast<const void*>(&prism::k_gemm8<false>));
      return launch_gemm_blocks(ctx, fn, tiles8, nsteps, nsplit8, w, d_X, M, d_Y, st, fixed);
    }
  }
  // GI weights (4-bit: K % 64 == 0, below 2 GiB; 8-bit: K % 512 == 0) always
  // take k_gemm_w4 or k_gemm8 above.
  if (w->gi) return fail(ctx, PRISM_HIP_ERR_SHAPE, "no GEMM kernel for this GI weight (%ux%u)", N, K);
  const uint32_t tiles = ((M + prism::GEMM_BM - 1) / prism::GEMM_BM) * ((N + prism::GEMM_BN - 1) / prism::GEMM_BN);
  const uint8_t* lut = w->lut();
  const uint8_t* idx = w->idx();
  const uint16_t* X = reinterpret_cast<const uint16_t*>(d_X);
  uint16_t* Y = reinterpret_cast<uint16_t*>(d_Y);
  void* args[] = {&lut, &idx, &X, &Y, &M, const_cast<uint32_t*>(&N), const_cast<uint32_t*>(&K)};
  const void* fn = bits == 4 ? reinterpret_cast<const void*>(&prism::k_gemm<4>)
                             : reinterpret_cast<const void*>(&prism::k_gemm<8>);
  HIP_TRY(ctx, launch_fn(fn, dim3(tiles), dim3(256), args, 0, st));
  return PRISM_HIP_OK;
}

int launch_decode(prism_hip_ctx* ctx, const prism_hip_weight* w, uint32_t row0, uint32_t nrows, void* d_out,
                  hipStream_t st) {
  const size_t total = (size_t)nrows * w->dim_n;
  if (total == 0) return PRISM_HIP_OK;
  size_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  const uint8_t* lut = w->lut();
  const uint8_t* idx = w->idx();
  uint32_t N = w->dim_m, K = w->dim_n;
  uint16_t* out = reinterpret_cast<uint16_t*>(d_out);
  uint32_t G = w->gi;
  void* args[] = {&lut, &idx, &N, &K, &row0, &nrows, &out, &G};
  const void* fn = w->bits == 8 ? (w->gi ? reinterpret_cast<const void*>(&prism::k_decode_rows<8, true>)
                                        : reinterpret_cast<const void*>(&prism::k_decode_rows<8>))
                   : w->gi      ? reinterpret_cast<const void*>(&prism::k_decode_rows<4, true>)
                                : reinterpret_cast<const void*>(&prism::k_decode_rows<4>);
  HIP_TRY(ctx, launch_fn(fn, dim3((unsigned)blocks), dim3(256), args, 0, st));
  return PRISM_HIP_OK;
}

// A 4-bit weight's LUT block and index rows in split-block form at dst_lut
// ([N][32] B) and dst_idx ([N][K/2] B), on stream st: copies, or for a GI
// weight the inverse regrouping.
int copy_split_rows(prism_hip_ctx* ctx, const prism_hip_weight* w, uint8_t* dst_lut, uint8_t* dst_idx,
                    hipStream_t st) {
  const uint32_t N = w->dim_m, K = w->dim_n;
  if (!w->gi) {
    HIP_TRY(ctx, hipMemcpyAsync(dst_lut, w->lut(), (size_t)N * 32, hipMemcpyDeviceToDevice, st));
    HIP_TRY(ctx, hipMemcpyAsync(dst_idx, w->idx(), (size_t)N * (K / 2), hipMemcpyDeviceToDevice, st));
    return PRISM_HIP_OK;
  }
  const size_t pieces = (size_t)N * (2 + K / 32);
  const unsigned grid = (unsigned)std::min<size_t>((pieces + 255) / 256, 16384);
  PRISM_LAUNCH(prism::k_gi_unpack, dim3(grid), dim3(256), 0, st, w->d, dst_lut, dst_idx, N, K, w->gi);
  HIP_TRY(ctx, hipGetLastError());
  return PRISM_HIP_OK;
}



}  // namespace

// =========================================================================
extern "C" {

const char* prism_hip_version(void) { return PRISM_HIP_VERSION; }

prism_hip_ctx* prism_hip_ctx_create(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    g_create_err = std::string("no HIP device: ") + hipGetErrorString(e);
    return nullptr;
  }
  if (device < 0 || device >= n) {
    g_create_err = "device index " + std::to_string(device) + " out of range (" + std::to_string(n) + " devices)";
    return nullptr;
  }
  DeviceGuard g(device);
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) {
    g_create_err = std::string("hipGetDeviceProperties: ") + hipGetErrorString(e);
    return nullptr;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    g_create_err = std::string("device is ") + prop.gcnArchName + ", this library is built for gfx950";
    return nullptr;
  }
  auto* ctx = new prism_hip_ctx;
  ctx->device = device;
  ctx->num_cu = prop.multiProcessorCount;
  ctx->lds_max = prop.sharedMemPerBlock;
  if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
    g_create_err = std::string("hipStreamCreate: ") + hipGetErrorString(e);
    delete ctx;
    return nullptr;
  }
  g_create_err.clear();
  return ctx;
}

void prism_hip_ctx_destroy(prism_hip_ctx* ctx) {
  if (!ctx) return;
  DeviceGuard g(ctx->device);
  for (prism_hip_weight* w : ctx->weights) w->ctx = nullptr;
  ctx->weights.clear();
  for (prism_hip_model* m : ctx->models) model_detach(m);
  ctx->models.clear();
  if (ctx->stream) {
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
  }
  if (ctx->d_stage) (void)hipFree(ctx->d_stage);
  if (ctx->d_upload) (void)hipFree(ctx->d_upload);
  chunk_release(ctx->carve);
  for (int i = 0; i < prism_hip_ctx::kRingSlots; i++) {
    if (ctx->ring[i]) (void)hipHostFree(ctx->ring[i]);
    if (ctx->ring_done[i]) (void)hipEventDestroy(ctx->ring_done[i]);
  }
  if (ctx->pool) {
    (void)hipDeviceSynchronize();  // scratch freed on other streams
    (void)hipMemPoolDestroy(ctx->pool);
  }
  delete ctx;
}

const char* prism_hip_last_error(const prism_hip_ctx* ctx) {
  return ctx ? ctx->err.c_str() : g_create_err.c_str();
}

const char* prism_hip_last_kernels(prism_hip_ctx* ctx) {
  if (!ctx) return "";
  if (ctx->kernels.empty() && !ctx->launched.empty()) {
    // device names of the recorded host functions, demangled and shortened
    // to the kernel's own name and template arguments
    std::string out, prev;
    int run = 0;
    auto flush = [&] {
      if (prev.empty()) return;
      if (!out.empty()) out += " + ";
      out += prev;
      if (run > 1) out += " x" + std::to_string(run);
    };
    for (const void* fn : ctx->launched) {
      const char* raw = hipKernelNameRefByPtr(fn, ctx->stream);
      std::string name = raw ? raw : "?";
      int st = 0;
      char* dem = raw ? abi::__cxa_demangle(raw, nullptr, nullptr, &st) : nullptr;
      if (dem && st == 0) name = dem;
      std::free(dem);
      size_t depth = 0, cut = std::string::npos;
      for (size_t i = 0; i < name.size(); i++) {  // the parameter list: the last top-level '('
        if (name[i] == '<') depth++;
        else if (name[i] == '>' && depth) depth--;
        else if (name[i] == '(' && depth == 0) cut = i;
      }
      if (cut != std::string::npos) name.resize(cut);
      if (name.compare(0, 5, "void ") == 0) name.erase(0, 5);
      for (size_t p; (p = name.find("prism::")) != std::string::npos;) name.erase(p, 7);
      if (name == prev) {
        run++;
      } else {
        flush();
        prev = name;
        run = 1;
      }
    }
    flush();
    ctx->kernels = out;
  }
  return ctx->kernels.c_str();
}

// Host payloads go through the pinned ring (stage_h2d); device payloads
// are copied device-to-device.  GI weights are regrouped on the device
// from a split-block copy (the context's upload buffer for host payloads).
// `async`: return once the copies are enqueued on the context stream.
static prism_hip_weight* upload_impl(prism_hip_ctx* ctx, const void* src, bool src_dev, size_t bytes, uint32_t dm,
                                     uint32_t dn, uint32_t bits, uint32_t layout, bool async = false) {
  if (!ctx) return nullptr;
  if (!src) {
    fail(ctx, PRISM_HIP_ERR_NULL, "payload is NULL");
    return nullptr;
  }
  if (check_shape(ctx, dm, dn, bits, layout, bytes) != PRISM_HIP_OK) return nullptr;
  DeviceGuard g(ctx->device);
  auto* w = new prism_hip_weight;
  w->ctx = ctx;
  w->device = ctx->device;
  w->dim_m = dm;
  w->dim_n = dn;
  w->bits = bits;
  w->layout = layout;
  w->bytes = bytes;
  w->gi = gi_rows(ctx, dm, dn, bits);
  auto bail = [&](int rc) -> prism_hip_weight* {
    (void)rc;
    if (w->chunk) {
      (void)hipStreamSynchronize(ctx->stream);
      chunk_release(w->chunk);
    }
    delete w;
    return nullptr;
  };
  int rc = weight_alloc(ctx, w->gi ? prism::gi_bytes(w->gi, dm, dn, bits) : bytes, &w->d, &w->chunk);
  if (rc != PRISM_HIP_OK) return bail(rc);
  hipError_t e = hipSuccess;
  const void* s = src;
  if (!w->gi) {
    if (src_dev) {
      e = hipMemcpyAsync(w->d, src, bytes, hipMemcpyDeviceToDevice, ctx->stream);
      if (e != hipSuccess) rc = fail(ctx, PRISM_HIP_ERR_DEVICE, "weight upload: %s", hipGetErrorString(e));
    } else {
      rc = stage_h2d(ctx, w->d, src, bytes);
    }
  } else {
    if (!src_dev) {
      rc = ensure_upload_stage(ctx, bytes);
      if (rc == PRISM_HIP_OK) rc = stage_h2d(ctx, ctx->d_upload, src, bytes);
      s = ctx->d_upload;
    }
    if (rc == PRISM_HIP_OK) {
      const size_t pieces = prism::gi_bytes(w->gi, dm, dn, bits) / 16;
      const unsigned grid = (unsigned)std::min<size_t>((pieces + 255) / 256, 16384);
      PRISM_LAUNCH(prism::k_gi_pack, dim3(grid), dim3(256), 0, ctx->stream,
                         reinterpret_cast<const uint8_t*>(s), w->d, dm, dn, w->gi, bits);
      e = hipGetLastError();
      if (e != hipSuccess) rc = fail(ctx, PRISM_HIP_ERR_DEVICE, "GI pack: %s", hipGetErrorString(e));
    }
  }
  if (rc == PRISM_HIP_OK && (!async || src_dev)) {
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) rc = fail(ctx, PRISM_HIP_ERR_DEVICE, "weight upload (%zu bytes): %s", bytes, hipGetErrorString(e));
  }
  if (rc != PRISM_HIP_OK) return bail(rc);
  ctx->weights.insert(w);
  ctx->err.clear();
  return w;
}

prism_hip_weight* prism_hip_weight_upload(prism_hip_ctx* ctx, const uint8_t* payload, size_t bytes, uint32_t dim_m,
                                          uint32_t dim_n, uint32_t bits, uint32_t layout) {
  return upload_impl(ctx, payload, false, bytes, dim_m, dim_n, bits, layout);
}

prism_hip_weight* prism_hip_weight_upload_async(prism_hip_ctx* ctx, const uint8_t* payload, size_t bytes,
                                                uint32_t dim_m, uint32_t dim_n, uint32_t bits, uint32_t layout) {
  return upload_impl(ctx, payload, false, bytes, dim_m, dim_n, bits, layout, true);
}

prism_hip_weight* prism_hip_weight_upload_dev(prism_hip_ctx* ctx, const void* d_payload, size_t bytes, uint32_t dim_m,
                                              uint32_t dim_n, uint32_t bits, uint32_t layout) {
  return upload_impl(ctx, d_payload, true, bytes, dim_m, dim_n, bits, layout);
}

int prism_hip_ctx_synchronize(prism_hip_ctx* ctx) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  DeviceGuard g(ctx->device);
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

void prism_hip_weight_free(prism_hip_weight* w) {
  if (!w) return;
  DeviceGuard g(w->device);
  if (w->ctx) w->ctx->weights.erase(w);
  chunk_release(w->chunk);  // the chunk's last weight frees it (hipFree waits for work still using it)
  delete w;
}

int prism_hip_weight_info(const prism_hip_weight* w, uint32_t* dim_m, uint32_t* dim_n, uint32_t* bits, size_t* bytes) {
  if (!w) return PRISM_HIP_ERR_NULL;
  if (dim_m) *dim_m = w->dim_m;
  if (dim_n) *dim_n = w->dim_n;
  if (bits) *bits = w->bits;
  if (bytes) *bytes = w->bytes;
  return PRISM_HIP_OK;
}

// ---- GEMV
int prism_hip_gemv_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_x, uint32_t batch, void* d_y,
                       void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!d_x || !d_y) return fail(ctx, PRISM_HIP_ERR_NULL, "x or y is NULL");
  if (batch == 0) return PRISM_HIP_OK;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_gemv(ctx, w, nullptr, d_x, batch, d_y, pick_stream(ctx, stream));
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_gemv(prism_hip_ctx* ctx, const prism_hip_weight* w, const uint16_t* x, uint32_t batch, uint16_t* y) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!x || !y) return fail(ctx, PRISM_HIP_ERR_NULL, "x or y is NULL");
  if (batch == 0) return PRISM_HIP_OK;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t xb = (size_t)batch * w->dim_n * 2, yb = (size_t)batch * w->dim_m * 2;
  const size_t xoff = 0, yoff = (xb + 255) & ~(size_t)255;
  if ((rc = ensure_stage(ctx, yoff + yb))) return rc;
  uint8_t* st = reinterpret_cast<uint8_t*>(ctx->d_stage);
  HIP_TRY(ctx, hipMemcpyAsync(st + xoff, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = launch_gemv(ctx, w, nullptr, st + xoff, batch, st + yoff, ctx->stream))) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(y, st + yoff, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- gate_up + SwiGLU
static int check_pair(prism_hip_ctx* ctx, const prism_hip_weight* g, const prism_hip_weight* u) {
  int rc = check_weight(ctx, g);
  if (rc) return rc;
  if ((rc = check_weight(ctx, u))) return rc;
  if (g->dim_m != u->dim_m || g->dim_n != u->dim_n || g->bits != u->bits)
    return fail(ctx, PRISM_HIP_ERR_MISMATCH, "gate %ux%u/%u-bit and up %ux%u/%u-bit differ", g->dim_m, g->dim_n,
                g->bits, u->dim_m, u->dim_n, u->bits);
  return PRISM_HIP_OK;
}

int prism_hip_gateup_swiglu_dev(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                                const void* d_x, void* d_y, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_pair(ctx, gate, up);
  if (rc) return rc;
  if (!d_x || !d_y) return fail(ctx, PRISM_HIP_ERR_NULL, "x or y is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_gemv(ctx, gate, up, d_x, 1, d_y, pick_stream(ctx, stream));
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_gateup_swiglu(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                            const uint16_t* x, uint16_t* y) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_pair(ctx, gate, up);
  if (rc) return rc;
  if (!x || !y) return fail(ctx, PRISM_HIP_ERR_NULL, "x or y is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t xb = (size_t)gate->dim_n * 2, yb = (size_t)gate->dim_m * 2;
  const size_t yoff = (xb + 255) & ~(size_t)255;
  if ((rc = ensure_stage(ctx, yoff + yb))) return rc;
  uint8_t* st = reinterpret_cast<uint8_t*>(ctx->d_stage);
  HIP_TRY(ctx, hipMemcpyAsync(st, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = launch_gemv(ctx, gate, up, st, 1, st + yoff, ctx->stream))) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(y, st + yoff, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- gate and up without the activation: two outputs
int prism_hip_gate_up_dev(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up,
                          const void* d_x, void* d_gate_out, void* d_up_out, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_pair(ctx, gate, up);
  if (rc) return rc;
  if (!d_x || !d_gate_out || !d_up_out) return fail(ctx, PRISM_HIP_ERR_NULL, "x or an output is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_gemv(ctx, gate, up, d_x, 1, d_gate_out, pick_stream(ctx, stream), d_up_out);
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_gate_up(prism_hip_ctx* ctx, const prism_hip_weight* gate, const prism_hip_weight* up, const uint16_t* x,
                      uint16_t* gate_out, uint16_t* up_out) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_pair(ctx, gate, up);
  if (rc) return rc;
  if (!x || !gate_out || !up_out) return fail(ctx, PRISM_HIP_ERR_NULL, "x or an output is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t xb = (size_t)gate->dim_n * 2, yb = (size_t)gate->dim_m * 2;
  const size_t yoff = (xb + 255) & ~(size_t)255, y2off = yoff + ((yb + 255) & ~(size_t)255);
  if ((rc = ensure_stage(ctx, y2off + yb))) return rc;
  uint8_t* st = reinterpret_cast<uint8_t*>(ctx->d_stage);
  HIP_TRY(ctx, hipMemcpyAsync(st, x, xb, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = launch_gemv(ctx, gate, up, st, 1, st + yoff, ctx->stream, st + y2off))) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(gate_out, st + yoff, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipMemcpyAsync(up_out, st + y2off, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- GEMM
int prism_hip_gemm_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_X, uint32_t M, void* d_Y,
                       void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!d_X || !d_Y) return fail(ctx, PRISM_HIP_ERR_NULL, "X or Y is NULL");
  if (M == 0) return PRISM_HIP_OK;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_gemm(ctx, w, d_X, M, d_Y, pick_stream(ctx, stream));
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_gemm_dev_noalloc(prism_hip_ctx* ctx, const prism_hip_weight* w, const void* d_X, uint32_t M,
                               void* d_Y, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!d_X || !d_Y) return fail(ctx, PRISM_HIP_ERR_NULL, "X or Y is NULL");
  if (M == 0) return PRISM_HIP_OK;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  if (!ctx->scratch) {
    const hipError_t e = device_scratch(ctx->device, &ctx->scratch);
    if (e != hipSuccess)
      return fail(ctx, PRISM_HIP_ERR_DEVICE, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  }
  rc = launch_gemm(ctx, w, d_X, M, d_Y, pick_stream(ctx, stream), ctx->scratch);
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_gemm(prism_hip_ctx* ctx, const prism_hip_weight* w, const uint16_t* X, uint32_t M, uint16_t* Y) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!X || !Y) return fail(ctx, PRISM_HIP_ERR_NULL, "X or Y is NULL");
  if (M == 0) return PRISM_HIP_OK;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t xb = (size_t)M * w->dim_n * 2, yb = (size_t)M * w->dim_m * 2;
  const size_t yoff = (xb + 255) & ~(size_t)255;
  if ((rc = ensure_stage(ctx, yoff + yb))) return rc;
  uint8_t* st = reinterpret_cast<uint8_t*>(ctx->d_stage);
  HIP_TRY(ctx, hipMemcpyAsync(st, X, xb, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = launch_gemm(ctx, w, st, M, st + yoff, ctx->stream))) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(Y, st + yoff, yb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- decode
int prism_hip_decode_rows_dev(prism_hip_ctx* ctx, const prism_hip_weight* w, uint32_t row0, uint32_t nrows,
                              void* d_out, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!d_out) return fail(ctx, PRISM_HIP_ERR_NULL, "out is NULL");
  if (row0 > w->dim_m || nrows > w->dim_m - row0)
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "rows [%u, %u) outside 0..%u", row0, row0 + nrows, w->dim_m);
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_decode(ctx, w, row0, nrows, d_out, pick_stream(ctx, stream));
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

int prism_hip_lut_embed(prism_hip_ctx* ctx, const prism_hip_weight* w, uint32_t token, uint16_t* out) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  int rc = check_weight(ctx, w);
  if (rc) return rc;
  if (!out) return fail(ctx, PRISM_HIP_ERR_NULL, "out is NULL");
  if (token >= w->dim_m) {  // evaluator.rs:182-184: out-of-range token -> zeros
    std::memset(out, 0, (size_t)w->dim_n * 2);
    ctx->err.clear();
    return PRISM_HIP_OK;
  }
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t ob = (size_t)w->dim_n * 2;
  if ((rc = ensure_stage(ctx, ob))) return rc;
  if ((rc = launch_decode(ctx, w, token, 1, ctx->d_stage, ctx->stream))) return rc;
  HIP_TRY(ctx, hipMemcpyAsync(out, ctx->d_stage, ob, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- measurement: the read floor
int prism_hip_stream_read_dev(prism_hip_ctx* ctx, const void* d_buf, size_t bytes, void* d_sink, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  if (!d_buf || !d_sink) return fail(ctx, PRISM_HIP_ERR_NULL, "buffer or sink is NULL");
  if (bytes == 0) return PRISM_HIP_OK;
  if (bytes >= (1ull << 31)) return fail(ctx, PRISM_HIP_ERR_SIZE, "%zu bytes: at most 2 GiB - 1 per call", bytes);
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const unsigned grid = (unsigned)((bytes + prism::kStreamBytesPerBlock - 1) / prism::kStreamBytesPerBlock);
  PRISM_LAUNCH(prism::k_stream_read, dim3(grid), dim3(64), 0, pick_stream(ctx, stream),
                     reinterpret_cast<const uint8_t*>(d_buf), (uint32_t)bytes, reinterpret_cast<uint32_t*>(d_sink));
  HIP_TRY(ctx, hipGetLastError());
  ctx->err.clear();
  return PRISM_HIP_OK;
}

// ---- measurement: one dependent launch, and the matrix cores' rate
int prism_hip_launch_empty_dev(prism_hip_ctx* ctx, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  PRISM_LAUNCH(prism::k_launch_empty, dim3(1), dim3(64), 0, pick_stream(ctx, stream));
  HIP_TRY(ctx, hipGetLastError());
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_mfma_probe_dev(prism_hip_ctx* ctx, uint32_t groups, uint32_t iters, void* d_sink, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  if (!d_sink) return fail(ctx, PRISM_HIP_ERR_NULL, "sink is NULL");
  if (groups == 0 || groups > 65536) return fail(ctx, PRISM_HIP_ERR_SIZE, "%u workgroups: 1..65536", groups);
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  PRISM_LAUNCH(prism::k_mfma_probe, dim3(groups), dim3(256), 0, pick_stream(ctx, stream), iters,
               reinterpret_cast<float*>(d_sink));
  HIP_TRY(ctx, hipGetLastError());
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_issue_probe_dev(prism_hip_ctx* ctx, uint32_t op, uint32_t groups, uint32_t waves_per_simd,
                              uint32_t iters, void* d_sink, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  if (!d_sink) return fail(ctx, PRISM_HIP_ERR_NULL, "sink is NULL");
  if (op > 3) return fail(ctx, PRISM_HIP_ERR_SHAPE, "instruction kind %u: 0..3", op);
  if (waves_per_simd != 1 && waves_per_simd != 2 && waves_per_simd != 4)
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "%u waves per SIMD: 1, 2 or 4", waves_per_simd);
  if (groups == 0 || groups > 65536) return fail(ctx, PRISM_HIP_ERR_SIZE, "%u workgroups: 1..65536", groups);
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const dim3 block(256 * waves_per_simd);
  hipStream_t st = pick_stream(ctx, stream);
  float* sink = reinterpret_cast<float*>(d_sink);
  switch (op) {
    case 0: PRISM_LAUNCH(prism::k_issue_probe<0>, dim3(groups), block, 0, st, iters, sink); break;
    case 1: PRISM_LAUNCH(prism::k_issue_probe<1>, dim3(groups), block, 0, st, iters, sink); break;
    case 2: PRISM_LAUNCH(prism::k_issue_probe<2>, dim3(groups), block, 0, st, iters, sink); break;
    default: PRISM_LAUNCH(prism::k_issue_probe<3>, dim3(groups), block, 0, st, iters, sink); break;
  }
  HIP_TRY(ctx, hipGetLastError());
  ctx->err.clear();
  return PRISM_HIP_OK;
}

}  // extern "C"

// GPU-resident decode step (prism_hip_model_*).

// ---- palette compiler
size_t prism_hip_palettize_bytes(uint32_t out_dim, uint32_t in_dim) {
  return (size_t)out_dim * 32 + (size_t)out_dim * ((in_dim + 1) / 2);
}

static int check_palettize(prism_hip_ctx* ctx, uint32_t k, const float* seeds, uint32_t nseeds,
                           prism::PaletteSeeds* ps) {
  if (k == 0 || k > (uint32_t)prism::kPaletteMaxK)
    return fail(ctx, PRISM_HIP_ERR_SHAPE, "palette size k=%u outside 1..%d (4-bit indices)", k, prism::kPaletteMaxK);
  *ps = prism::PaletteSeeds{};
  if (seeds) {
    if (nseeds == 0)  // the reference would index centroids[-1]
      return fail(ctx, PRISM_HIP_ERR_SHAPE, "seeds given with nseeds = 0");
    ps->n = std::min<uint32_t>(nseeds, prism::kPaletteMaxK);
    std::memcpy(ps->v, seeds, ps->n * sizeof(float));
  }
  return PRISM_HIP_OK;
}

// Rows run one wave each.  When a row's arrays fit the workgroup's LDS they
// live there; longer rows keep them in a stream-ordered workspace of at most
// kWsBytes per launch.
static int launch_palettize(prism_hip_ctx* ctx, const float* d_w, uint32_t out_dim, uint32_t in_dim, uint32_t k,
                            uint32_t max_iter, const prism::PaletteSeeds& seeds, uint8_t* d_payload,
                            hipStream_t st) {
  constexpr uint32_t kMaxGrid = 1u << 20;
  constexpr size_t kWsBytes = (size_t)256 << 20;
  uint8_t* lut = d_payload;
  uint8_t* idx = d_payload + (size_t)out_dim * 32;
  const size_t lds = prism::palette_row_bytes(in_dim);
  const size_t stat = 3 * prism::kPaletteMaxK * 4;
  if (lds + stat <= ctx->lds_max) {
    for (uint32_t r0 = 0; r0 < out_dim; r0 += kMaxGrid) {
      const uint32_t rows = std::min(kMaxGrid, out_dim - r0);
      PRISM_LAUNCH(prism::k_palettize<true>, dim3(rows), dim3(64), lds, st, d_w, in_dim, k, max_iter, seeds,
                         r0, nullptr, lut, idx);
      HIP_TRY(ctx, hipGetLastError());
    }
    return PRISM_HIP_OK;
  }
  const uint32_t chunk = (uint32_t)std::min<size_t>(kMaxGrid, std::max<size_t>(1, kWsBytes / lds));
  const size_t wsb = (size_t)std::min(chunk, out_dim) * lds;
  void* ws = nullptr;
  HIP_TRY(ctx, hipMallocAsync(&ws, wsb, st));
  for (uint32_t r0 = 0; r0 < out_dim; r0 += chunk) {
    const uint32_t rows = std::min(chunk, out_dim - r0);
    PRISM_LAUNCH(prism::k_palettize<false>, dim3(rows), dim3(64), 0, st, d_w, in_dim, k, max_iter, seeds,
                       r0, reinterpret_cast<float*>(ws), lut, idx);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      (void)hipFreeAsync(ws, st);
      return fail(ctx, PRISM_HIP_ERR_DEVICE, "k_palettize launch failed: %s", hipGetErrorString(e));
    }
  }
  HIP_TRY(ctx, hipFreeAsync(ws, st));
  return PRISM_HIP_OK;
}

int prism_hip_palettize(prism_hip_ctx* ctx, const float* w, uint32_t out_dim, uint32_t in_dim, uint32_t k,
                        uint32_t max_iter, const float* seeds, uint32_t nseeds, uint8_t* payload) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  prism::PaletteSeeds ps;
  int rc = check_palettize(ctx, k, seeds, nseeds, &ps);
  if (rc) return rc;
  if (out_dim == 0) return PRISM_HIP_OK;
  if (!payload || (!w && in_dim)) return fail(ctx, PRISM_HIP_ERR_NULL, "weights or payload is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  const size_t wb = (size_t)out_dim * in_dim * 4, pb = prism_hip_palettize_bytes(out_dim, in_dim);
  const size_t poff = (wb + 255) & ~(size_t)255;
  if ((rc = ensure_stage(ctx, poff + pb))) return rc;
  uint8_t* st = reinterpret_cast<uint8_t*>(ctx->d_stage);
  if (wb) HIP_TRY(ctx, hipMemcpyAsync(st, w, wb, hipMemcpyHostToDevice, ctx->stream));
  if ((rc = launch_palettize(ctx, reinterpret_cast<const float*>(st), out_dim, in_dim, k, max_iter, ps, st + poff,
                             ctx->stream)))
    return rc;
  HIP_TRY(ctx, hipMemcpyAsync(payload, st + poff, pb, hipMemcpyDeviceToHost, ctx->stream));
  HIP_TRY(ctx, hipStreamSynchronize(ctx->stream));
  ctx->err.clear();
  return PRISM_HIP_OK;
}

int prism_hip_palettize_dev(prism_hip_ctx* ctx, const void* d_w, uint32_t out_dim, uint32_t in_dim, uint32_t k,
                            uint32_t max_iter, const float* seeds, uint32_t nseeds, void* d_payload, void* stream) {
  if (!ctx) return PRISM_HIP_ERR_NULL;
  prism::PaletteSeeds ps;
  int rc = check_palettize(ctx, k, seeds, nseeds, &ps);
  if (rc) return rc;
  if (out_dim == 0) return PRISM_HIP_OK;
  if (!d_payload || (!d_w && in_dim)) return fail(ctx, PRISM_HIP_ERR_NULL, "weights or payload is NULL");
  DeviceGuard g(ctx->device);
  LaunchLog log(ctx);
  rc = launch_palettize(ctx, reinterpret_cast<const float*>(d_w), out_dim, in_dim, k, max_iter, ps,
                        reinterpret_cast<uint8_t*>(d_payload), pick_stream(ctx, stream));
  if (rc == PRISM_HIP_OK) ctx->err.clear();
  return rc;
}

#include "model_step.hpp"
