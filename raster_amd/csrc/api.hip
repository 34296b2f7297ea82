// api.hip — the C ABI declared in include/rq.h.
//
// Handles (contexts, weights, buffers) live in process-wide registries guarded
// by one mutex, so a destroyed, double-freed or foreign handle is reported as
// RQ_ERR_HANDLE instead of being dereferenced. Errors carry a message in a
// thread-local string (rq_last_error).
#include <algorithm>
#include <atomic>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "rq_internal.h"

namespace rq {

// Device scratch of rq_qmatmul_noalloc: a file-scope array that every GPU the
// library runs on holds until the process ends. In host code `scratch` names a
// host-side stand-in, not device memory: its device address (one per device)
// comes from hipGetSymbolAddress at context creation and is kept in
// g_scratch_ptr; only that address is passed to kernels.
static constexpr size_t kNoAllocScratchBytes = (size_t)RQ_NOALLOC_SCRATCH_MAX;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static constexpr int kMaxDevices = 64;

// Timing events of one call: e[0], e[1] bracket the main kernel (for the
// bf16 GEMM: the packing pass's end and the GEMM's end); on calls whose
// partial sums a second kernel adds, e[2], e[3] bracket that kernel (n = 4).
// The call's time is the sum of its kernels' own durations, without the gap
// between them.
struct EvSet {
  hipEvent_t e[4] = {nullptr, nullptr, nullptr, nullptr};
  int n = 0;
};

struct Ctx {
  uint32_t magic;
  int device;
  int cu_count;
  int wave_size;
  int clock_khz;
  std::unordered_set<Weight*> weights;
  std::unordered_set<void*> buffers;
  // Per-stream scratch, grow-only, freed with the context: packed
  // activations, and the K-split partial sums. Calls on one stream run in
  // order, so a stream's buffers are never used by two kernels at once.
  struct StreamScratch {
    void* pack = nullptr;
    size_t pack_bytes = 0;
    void* red = nullptr;  // K-split partial sums
    size_t red_bytes = 0;
    void* attn = nullptr;  // split attention: the ranges' softmax records
    size_t attn_bytes = 0;
  };
  std::unordered_map<hipStream_t, StreamScratch> scratch;
  // Scratch buffers replaced by larger ones. A graph captured on a stream
  // keeps the addresses it was captured with, so a buffer that grew is kept
  // until the context is destroyed rather than freed: replaying such a graph
  // after a larger call still finds its memory. (Growth is by at least 25%
  // each time, so the retired buffers total at most four times the largest.)
  std::vector<void*> retired;
  // rocBLAS handle of the dense f32 GEMM entries, created on first use; the
  // mutex covers setting its stream and enqueueing one call
  void* blas = nullptr;
  std::mutex blas_mu;
  // Kernel timing (rq_ctx_set_kernel_timing): per timed call an event set (a
  // start / end pair per kernel, EvSet), waiting to be read, and a pool of
  // spares.
  std::atomic<bool> timing{false};
  std::mutex timing_mu;
  std::vector<EvSet> ev_pending, ev_pool;
};

static constexpr uint32_t kCtxMagic = 0x52514358u;     // "RQCX"
static constexpr uint32_t kWeightMagic = 0x52515754u;  // "RQWT"

static std::mutex g_mu;
static void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device (under g_mu)
static std::unordered_set<Ctx*> g_ctxs;
static std::unordered_set<Weight*> g_weights;
static thread_local std::string t_err;

static int fail(int status, const std::string& msg) {
  t_err = msg;
  return status;
}

static int hip_fail(hipError_t e, const char* what) {
  return fail(RQ_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define RQ_HIP(call, what)                   \
  do {                                       \
    hipError_t e_ = (call);                  \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

static bool live_ctx(Ctx* c) { return c && g_ctxs.count(c) && c->magic == kCtxMagic; }
static bool live_weight(Weight* w) { return w && g_weights.count(w) && w->magic == kWeightMagic; }

static int check_ctx(Ctx* c) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_ctx(c)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_ctx");
  return RQ_OK;
}

static int set_device(Ctx* c) {
  RQ_HIP(hipSetDevice(c->device), "hipSetDevice");
  return RQ_OK;
}

static int check_shape(int64_t out, int64_t in) {
  if (out <= 0 || in <= 0) return fail(RQ_ERR_SHAPE, "out and in must be positive");
  if (in % 32 != 0) return fail(RQ_ERR_SHAPE, "in=" + std::to_string(in) + " not a multiple of 32");
  if (in > (int64_t)1 << 30 || out > (int64_t)1 << 30) return fail(RQ_ERR_SHAPE, "dimension too large");
  return RQ_OK;
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Allocates the weight, uploads Raster's row-major codes/packed bytes and
// scales to a staging buffer and converts them to the chunked device layout.
static int make_weight(Ctx* c, int format, int scale_dtype, int64_t out, int64_t in, const void* qhost,
                       const void* shost, rq_weight* wout) {
  const int64_t npad = (out + 15) / 16 * 16;
  const size_t ssz = scale_dtype == RQ_F16 ? 2 : 4;
  const size_t qbytes_rm = (size_t)out * (size_t)(in / 32) * code_bytes(format);
  const size_t sbytes_rm = (size_t)out * (size_t)(in / 32) * ssz;
  const size_t qbytes = (size_t)npad * (size_t)(in / 32) * code_bytes(format);
  const size_t sbytes = (size_t)npad * (size_t)(in / 32) * ssz;
  const size_t sbytes_rb = (size_t)npad * (size_t)scale_nb8(in / 32) * ssz;
  const size_t total = align256(qbytes) + align256(sbytes) + align256(sbytes_rb);
  if (int s = set_device(c)) return s;
  void* base = nullptr;
  hipError_t e = hipMalloc(&base, total);
  if (e != hipSuccess || !base) {
    (void)hipGetLastError();
    return fail(RQ_ERR_OOM, "hipMalloc of " + std::to_string(total) + " bytes for weight failed");
  }
  void* stage = nullptr;
  e = hipMalloc(&stage, align256(qbytes_rm) + sbytes_rm);
  if (e != hipSuccess || !stage) {
    (void)hipGetLastError();
    (void)hipFree(base);
    return fail(RQ_ERR_OOM, "hipMalloc of the weight staging buffer failed");
  }
  Weight* w = new (std::nothrow) Weight();
  if (!w) {
    (void)hipFree(stage);
    (void)hipFree(base);
    return fail(RQ_ERR_OOM, "host allocation failed");
  }
  w->magic = kWeightMagic;
  w->format = format;
  w->scale_dtype = scale_dtype;
  w->device = c->device;
  w->out = out;
  w->in = in;
  w->npad = npad;
  w->base = base;
  w->q = static_cast<uint8_t*>(base);
  w->scales = static_cast<uint8_t*>(base) + align256(qbytes);
  w->scales_rb = static_cast<uint8_t*>(base) + align256(qbytes) + align256(sbytes);
  w->bytes = total;
  w->ctx = c;
  uint8_t* q_rm = static_cast<uint8_t*>(stage);
  uint8_t* s_rm = q_rm + align256(qbytes_rm);
  e = hipMemcpy(q_rm, qhost, qbytes_rm, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(s_rm, shost, sbytes_rm, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_chunk_weight(format, scale_dtype, q_rm, s_rm, out, in, npad, w->q, w->scales, w->scales_rb,
                                               nullptr);
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  (void)hipFree(stage);
  if (e != hipSuccess) {
    (void)hipFree(base);
    delete w;
    return hip_fail(e, "weight upload");
  }
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!live_ctx(c)) {
      (void)hipFree(base);
      delete w;
      return fail(RQ_ERR_HANDLE, "rq_ctx destroyed during weight creation");
    }
    g_weights.insert(w);
    c->weights.insert(w);
  }
  *wout = reinterpret_cast<rq_weight>(w);
  return RQ_OK;
}

static bool capturing(hipStream_t stream) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

static const char* kCaptureScratch =
    "this stream is being captured and its scratch is too small for this call: run the same (or a larger) "
    "call on the stream once before capturing";

// Replaces *buf (sized *have) by a fresh allocation of at least `bytes`
// (+25%). The old buffer is retired, not freed: kernels queued on the stream
// and graphs captured earlier may still use it (freed at rq_ctx_destroy).
// Caller holds g_mu.
static int regrow(Ctx* c, size_t bytes, void** buf, size_t* have) {
  const size_t want = bytes + bytes / 4;
  void* p = nullptr;
  if (hipMalloc(&p, want) != hipSuccess || !p) {
    (void)hipGetLastError();
    return fail(RQ_ERR_OOM, "hipMalloc of " + std::to_string(want) + " bytes of scratch failed");
  }
  if (*buf) c->retired.push_back(*buf);
  *buf = p;
  *have = want;
  return RQ_OK;
}

// The bf16 GEMM's packed-activation buffer for `stream`, at least `bytes`.
static int stream_pack(Ctx* c, hipStream_t stream, size_t bytes, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto& e = c->scratch[stream];
  if (e.pack_bytes < bytes) {
    if (capturing(stream)) return fail(RQ_ERR_SHAPE, kCaptureScratch);
    if (int s = regrow(c, bytes, &e.pack, &e.pack_bytes)) return s;
  }
  *out = e.pack;
  return RQ_OK;
}

// The K-split partial sums for `stream`: `part_bytes` (grow-only).
static int stream_split(Ctx* c, hipStream_t stream, size_t part_bytes, float** part) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto& e = c->scratch[stream];
  if (e.red_bytes < part_bytes) {
    if (capturing(stream)) return fail(RQ_ERR_SHAPE, kCaptureScratch);
    if (int s = regrow(c, part_bytes, &e.red, &e.red_bytes)) return s;
  }
  *part = static_cast<float*>(e.red);
  return RQ_OK;
}

// The split attention's range records for `stream`: `bytes` (grow-only).
static int stream_attn(Ctx* c, hipStream_t stream, size_t bytes, void** out) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto& e = c->scratch[stream];
  if (e.attn_bytes < bytes) {
    if (capturing(stream)) return fail(RQ_ERR_SHAPE, kCaptureScratch);
    if (int s = regrow(c, bytes, &e.attn, &e.attn_bytes)) return s;
  }
  *out = e.attn;
  return RQ_OK;
}

// Timing events for one call on `stream` (two kernels when `two`), or an empty
// set when timing is off or the stream is being captured.
static EvSet timing_set(Ctx* c, hipStream_t stream, bool two = false) {
  if (!c->timing.load(std::memory_order_relaxed)) return {};
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return {};
  std::lock_guard<std::mutex> lk(c->timing_mu);
  EvSet set;
  if (!c->ev_pool.empty()) {
    set = c->ev_pool.back();
    c->ev_pool.pop_back();
  } else {
    // timing-only events (no system-scope fence: nothing is synchronised through them)
    for (int i = 0; i < 4; i++) {
      if (hipEventCreateWithFlags(&set.e[i], hipEventDisableSystemFence) != hipSuccess) {
        for (int j = 0; j < i; j++) (void)hipEventDestroy(set.e[j]);
        return {};
      }
    }
  }
  set.n = two ? 4 : 2;
  return set;
}

static void timing_done(Ctx* c, EvSet set, bool launched) {
  if (!set.n) return;
  std::lock_guard<std::mutex> lk(c->timing_mu);
  (launched ? c->ev_pending : c->ev_pool).push_back(set);
}

static void timing_release(Ctx* c) {
  std::lock_guard<std::mutex> lk(c->timing_mu);
  for (auto* v : {&c->ev_pending, &c->ev_pool}) {
    for (auto& set : *v) {
      if (set.n) (void)hipEventSynchronize(set.e[set.n - 1]);
      for (hipEvent_t e : set.e) (void)hipEventDestroy(e);
    }
    v->clear();
  }
}

static void free_weight_locked(Weight* w) {
  (void)hipSetDevice(w->device);
  (void)hipFree(w->base);
  w->magic = 0;
  g_weights.erase(w);
  delete w;
}

}  // namespace rq

using namespace rq;

extern "C" {

int rq_version(void) { return RQ_VERSION; }

const char* rq_status_string(int s) {
  switch (s) {
    case RQ_OK: return "ok";
    case RQ_ERR_SHAPE: return "bad shape";
    case RQ_ERR_DTYPE: return "unsupported dtype or format";
    case RQ_ERR_NULL: return "null pointer";
    case RQ_ERR_OOM: return "out of device memory";
    case RQ_ERR_HIP: return "HIP runtime error";
    case RQ_ERR_HANDLE: return "invalid handle";
    case RQ_ERR_DEVICE: return "no gfx950 device";
    default: return "unknown status";
  }
}

const char* rq_last_error(void) { return t_err.c_str(); }

int rq_ctx_create(int device, rq_ctx* out) {
  if (!out) return fail(RQ_ERR_NULL, "out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return fail(RQ_ERR_DEVICE, "no HIP device visible");
  }
  if (device < 0 || device >= n) return fail(RQ_ERR_DEVICE, "device id out of range");
  hipDeviceProp_t p;
  RQ_HIP(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
  if (std::string(p.gcnArchName).rfind("gfx950", 0) != 0)
    return fail(RQ_ERR_DEVICE, std::string("device is ") + p.gcnArchName + ", librq is built for gfx950");
  if (device >= kMaxDevices) return fail(RQ_ERR_DEVICE, "device id above the library's device table");
  {
    // once per device, with the device current: the address of this device's
    // copy of `scratch` (rq_qmatmul_noalloc)
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch_ptr[device]) {
      RQ_HIP(hipSetDevice(device), "hipSetDevice");
      void* ptr = nullptr;
      RQ_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
      if (!ptr) return fail(RQ_ERR_HIP, "hipGetSymbolAddress(scratch) returned NULL");
      g_scratch_ptr[device] = ptr;
    }
  }
  Ctx* c = new (std::nothrow) Ctx();
  if (!c) return fail(RQ_ERR_OOM, "host allocation failed");
  c->magic = kCtxMagic;
  c->device = device;
  c->cu_count = p.multiProcessorCount;
  c->wave_size = p.warpSize;
  c->clock_khz = p.clockRate;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    g_ctxs.insert(c);
  }
  *out = reinterpret_cast<rq_ctx>(c);
  return RQ_OK;
}

int rq_ctx_destroy(rq_ctx h) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_ctx(c)) return fail(RQ_ERR_HANDLE, "unknown or already destroyed rq_ctx");
  (void)hipSetDevice(c->device);
  for (Weight* w : c->weights) free_weight_locked(w);
  for (void* b : c->buffers) (void)hipFree(b);
  for (auto& kv : c->scratch) {
    (void)hipFree(kv.second.pack);
    (void)hipFree(kv.second.red);
    (void)hipFree(kv.second.attn);
  }
  for (void* p : c->retired) (void)hipFree(p);
  timing_release(c);
  {
    std::lock_guard<std::mutex> bl(c->blas_mu);
    dense_destroy(c->blas);
    c->blas = nullptr;
  }
  c->magic = 0;
  g_ctxs.erase(c);
  delete c;
  return RQ_OK;
}

int rq_ctx_device_info(rq_ctx h, int* cu_count, int* wave_size, int* clock_khz) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (cu_count) *cu_count = c->cu_count;
  if (wave_size) *wave_size = c->wave_size;
  if (clock_khz) *clock_khz = c->clock_khz;
  return RQ_OK;
}

int rq_ctx_set_kernel_timing(rq_ctx h, int enable) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (int s = set_device(c)) return s;
  c->timing.store(enable != 0);
  if (!enable) timing_release(c);
  return RQ_OK;
}

int rq_ctx_kernel_time(rq_ctx h, double* total_ms, int64_t* launches) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!total_ms || !launches) return fail(RQ_ERR_NULL, "total_ms or launches is NULL");
  if (int s = set_device(c)) return s;
  std::lock_guard<std::mutex> lk(c->timing_mu);
  double sum = 0.0;
  int64_t n = 0;
  hipError_t err = hipSuccess;
  for (auto& set : c->ev_pending) {
    float ms = 0.0f, ms2 = 0.0f;
    hipError_t e = hipEventSynchronize(set.e[set.n - 1]);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, set.e[0], set.e[1]);
    if (e == hipSuccess && set.n == 4) e = hipEventElapsedTime(&ms2, set.e[2], set.e[3]);
    if (e == hipSuccess) {
      sum += (double)ms + (double)ms2;
      n++;
    } else if (err == hipSuccess) {
      err = e;
    }
    set.n = 0;
    c->ev_pool.push_back(set);
  }
  c->ev_pending.clear();
  *total_ms = sum;
  *launches = n;
  if (err != hipSuccess) return hip_fail(err, "reading kernel timing events");
  return RQ_OK;
}

int rq_buf_alloc(rq_ctx h, size_t bytes, void** dptr) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!dptr) return fail(RQ_ERR_NULL, "dptr is NULL");
  *dptr = nullptr;
  if (bytes == 0) return fail(RQ_ERR_SHAPE, "zero-byte buffer");
  if (int s = set_device(c)) return s;
  void* p = nullptr;
  if (hipMalloc(&p, bytes) != hipSuccess || !p) {
    (void)hipGetLastError();
    return fail(RQ_ERR_OOM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
  }
  std::lock_guard<std::mutex> lk(g_mu);
  c->buffers.insert(p);
  *dptr = p;
  return RQ_OK;
}

int rq_buf_free(rq_ctx h, void* dptr) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_ctx(c)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_ctx");
  if (!dptr || !c->buffers.count(dptr)) return fail(RQ_ERR_HANDLE, "pointer is not a live rq_buf of this context");
  (void)hipSetDevice(c->device);
  c->buffers.erase(dptr);
  RQ_HIP(hipFree(dptr), "hipFree");
  return RQ_OK;
}

int rq_upload(rq_ctx h, void* dst, const void* src, size_t bytes, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!dst || !src) return fail(RQ_ERR_NULL, "NULL pointer");
  if (int s = set_device(c)) return s;
  RQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream), "hipMemcpyAsync H2D");
  RQ_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  return RQ_OK;
}

int rq_download(rq_ctx h, void* dst, const void* src, size_t bytes, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!dst || !src) return fail(RQ_ERR_NULL, "NULL pointer");
  if (int s = set_device(c)) return s;
  RQ_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream), "hipMemcpyAsync D2H");
  RQ_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  return RQ_OK;
}

int rq_stream_create(rq_ctx h, void** stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!stream) return fail(RQ_ERR_NULL, "stream is NULL");
  if (int s = set_device(c)) return s;
  hipStream_t st;
  RQ_HIP(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
  *stream = (void*)st;
  return RQ_OK;
}

int rq_stream_destroy(rq_ctx h, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!stream) return fail(RQ_ERR_NULL, "stream is NULL");
  RQ_HIP(hipStreamDestroy((hipStream_t)stream), "hipStreamDestroy");
  return RQ_OK;
}

int rq_sync(rq_ctx h, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (int s = set_device(c)) return s;
  RQ_HIP(hipStreamSynchronize((hipStream_t)stream), "hipStreamSynchronize");
  return RQ_OK;
}

int rq_weight_create_q8(rq_ctx h, const int8_t* codes, const float* scales, int64_t out, int64_t in,
                        rq_weight* w) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!codes || !scales || !w) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  return make_weight(c, RQ_Q8_0, RQ_F32, out, in, codes, scales, w);
}

int rq_weight_create_q8_packed(rq_ctx h, const int32_t* wp, const float* ws, int64_t out, int64_t in,
                               rq_weight* w) {
  // four little-endian int8 lanes per word: the words' bytes are the codes in order
  return rq_weight_create_q8(h, reinterpret_cast<const int8_t*>(wp), ws, out, in, w);
}

int rq_weight_create_q4(rq_ctx h, const uint8_t* packed, const void* scales, int scale_dtype, int64_t out,
                        int64_t in, rq_weight* w) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!packed || !scales || !w) return fail(RQ_ERR_NULL, "NULL argument");
  if (scale_dtype != RQ_F32 && scale_dtype != RQ_F16) return fail(RQ_ERR_DTYPE, "Q4 scales must be f32 or f16");
  if (int s = check_shape(out, in)) return s;
  return make_weight(c, RQ_Q4_0, scale_dtype, out, in, packed, scales, w);
}

int rq_weight_create_x8(rq_ctx h, const uint8_t* wqi, const float* wsi, int nibble, int64_t out, int64_t in,
                        rq_weight* w) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!wqi || !wsi || !w) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  if (out % 8 != 0) return fail(RQ_ERR_SHAPE, "x8 layout needs out % 8 == 0");
  // Invert the column interleave of raster/compiler/core/layout.clj:246-286
  // (tile 8, k-group 4, 8 input groups per 32-block).
  const int64_t nb = in / 32, ng = out / 8;
  std::vector<float> ws((size_t)(out * nb));
  for (int64_t g = 0; g < ng; g++)
    for (int64_t b = 0; b < nb; b++)
      for (int r = 0; r < 8; r++) ws[(size_t)((g * 8 + r) * nb + b)] = wsi[g * nb * 8 + b * 8 + r];
  if (nibble) {
    std::vector<uint8_t> packed((size_t)(out * in / 2));
    for (int64_t g = 0; g < ng; g++)
      for (int64_t b = 0; b < nb; b++)
        for (int ig = 0; ig < 8; ig++)
          for (int j = 0; j < 16; j++) {
            const uint8_t byte = wqi[g * nb * 128 + b * 128 + ig * 16 + j];
            const int e = ig * 4 + j % 4;           // element of the block
            const int64_t col = g * 8 + j / 4;      // low nibble column; high = col + 4
            const int64_t cols[2] = {col, col + 4};
            const uint8_t nibs[2] = {(uint8_t)(byte & 0xF), (uint8_t)(byte >> 4)};
            for (int t = 0; t < 2; t++) {
              uint8_t& dst = packed[(size_t)(cols[t] * (in / 2) + b * 16 + (e < 16 ? e : e - 16))];
              dst = e < 16 ? (uint8_t)((dst & 0xF0) | nibs[t]) : (uint8_t)((dst & 0x0F) | (nibs[t] << 4));
            }
          }
    return make_weight(c, RQ_Q4_0, RQ_F32, out, in, packed.data(), ws.data(), w);
  }
  // byte-direct unsigned codes with zero-point 128 -> signed codes (u - 128)
  std::vector<int8_t> codes((size_t)(out * in));
  for (int64_t g = 0; g < ng; g++)
    for (int64_t b = 0; b < nb; b++)
      for (int ig = 0; ig < 8; ig++)
        for (int j = 0; j < 32; j++) {
          const uint8_t u = wqi[g * nb * 256 + b * 256 + ig * 32 + j];
          const int64_t row = g * 8 + j / 4;
          const int e = ig * 4 + j % 4;
          codes[(size_t)(row * in + b * 32 + e)] = (int8_t)((int)u - 128);
        }
  return make_weight(c, RQ_Q8_0, RQ_F32, out, in, codes.data(), ws.data(), w);
}

int rq_weight_destroy(rq_weight h) {
  Weight* w = reinterpret_cast<Weight*>(h);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_weight(w)) return fail(RQ_ERR_HANDLE, "unknown or already destroyed rq_weight");
  if (live_ctx(w->ctx)) w->ctx->weights.erase(w);
  free_weight_locked(w);
  return RQ_OK;
}

// K-quant weight from host arrays already in the resident order: codes
// (qbytes), super-block scales (sbytes), sub-block scales (ubytes).
static int make_weight_k(Ctx* c, int format, int64_t out, int64_t in, const void* codes, size_t qbytes,
                         const void* sup, size_t sbytes, const void* sub, size_t ubytes, rq_weight* wout) {
  if (int s = set_device(c)) return s;
  const size_t total = align256(qbytes) + align256(sbytes) + align256(ubytes);
  void* base = nullptr;
  hipError_t e = hipMalloc(&base, total);
  if (e != hipSuccess || !base) {
    (void)hipGetLastError();
    return fail(RQ_ERR_OOM, "hipMalloc of " + std::to_string(total) + " bytes for weight failed");
  }
  Weight* w = new (std::nothrow) Weight();
  if (!w) {
    (void)hipFree(base);
    return fail(RQ_ERR_OOM, "host allocation failed");
  }
  w->magic = kWeightMagic;
  w->format = format;
  w->scale_dtype = RQ_F32;
  w->device = c->device;
  w->out = out;
  w->in = in;
  w->npad = out;
  w->base = base;
  w->q = static_cast<uint8_t*>(base);
  w->scales = static_cast<uint8_t*>(base) + align256(qbytes);
  w->scales_rb = nullptr;
  w->sub_scales = static_cast<uint8_t*>(base) + align256(qbytes) + align256(sbytes);
  w->bytes = total;
  w->ctx = c;
  e = hipMemcpy(w->q, codes, qbytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(w->scales, sup, sbytes, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(w->sub_scales, sub, ubytes, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(base);
    delete w;
    return hip_fail(e, "weight upload");
  }
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!live_ctx(c)) {
      (void)hipFree(base);
      delete w;
      return fail(RQ_ERR_HANDLE, "rq_ctx destroyed during weight creation");
    }
    g_weights.insert(w);
    c->weights.insert(w);
  }
  *wout = reinterpret_cast<rq_weight>(w);
  return RQ_OK;
}

static int check_shape_k(int format, int64_t out, int64_t in) {
  if (int s = check_shape(out, in)) return s;
  if (in % 256 != 0) return fail(RQ_ERR_SHAPE, "K-quants need in % 256 == 0 (super-blocks of 256)");
  // four activation rows of codes, sub-block sums and scales staged in LDS:
  // in <= 32768 for Q4_K, 32256 for Q6_K
  if (in > (int64_t)1 << 15 || kquant_gemv_lds(format, in, 4) > 163840)
    return fail(RQ_ERR_SHAPE, "K-quant in too large (activations staged in LDS: at most 32768 for Q4_K, "
                              "32256 for Q6_K)");
  return RQ_OK;
}

int rq_weight_create_q4k(rq_ctx h, const uint8_t* wq, const float* da, const float* db, const uint8_t* aq,
                         const int8_t* bq, int64_t out, int64_t in, rq_weight* w) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!wq || !da || !db || !aq || !bq || !w) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape_k(RQ_Q4_K, out, in)) return s;
  const int64_t nsb = out * (in / 256), nsub = out * (in / 32);
  std::vector<float> sup((size_t)(2 * nsb));
  for (int64_t i = 0; i < nsb; i++) {
    sup[(size_t)(2 * i)] = da[i];
    sup[(size_t)(2 * i + 1)] = db[i];
  }
  std::vector<uint16_t> sub((size_t)nsub);
  for (int64_t i = 0; i < nsub; i++) sub[(size_t)i] = (uint16_t)(aq[i] | ((uint16_t)(uint8_t)bq[i] << 8));
  return make_weight_k(c, RQ_Q4_K, out, in, wq, (size_t)(out * in / 2), sup.data(), sup.size() * 4, sub.data(),
                       sub.size() * 2, w);
}

int rq_weight_create_q6k(rq_ctx h, const uint8_t* wq, const int8_t* sc, const float* ds, int64_t out, int64_t in,
                         rq_weight* w) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!wq || !sc || !ds || !w) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape_k(RQ_Q6_K, out, in)) return s;
  // the device keeps the 6-bit codes packed, 12 bytes per 16-code sub-block
  // (the layout unpack_q6k in kquant.hip reads): 3/4 of Raster's byte per code
  const size_t n = (size_t)out * (size_t)in;
  std::vector<uint8_t> packed;
  try {
    packed.resize(n / 16 * 12);
  } catch (const std::bad_alloc&) {
    return fail(RQ_ERR_OOM, "host allocation failed");
  }
  uint8_t bad = 0;
  for (size_t sb = 0; sb < n / 16; sb++) {
    const uint8_t* q = wq + 16 * sb;
    uint8_t* d = packed.data() + 12 * sb;
    for (int j = 0; j < 16; j++) bad |= q[j];
    for (int j = 0; j < 8; j++) d[j] = (uint8_t)((q[j] & 15) | ((q[j + 8] & 15) << 4));
    for (int j = 0; j < 4; j++)
      d[8 + j] = (uint8_t)((q[j] >> 4) | ((q[j + 4] >> 4) << 2) | ((q[j + 8] >> 4) << 4) | ((q[j + 12] >> 4) << 6));
  }
  if (bad & 0xC0) return fail(RQ_ERR_SHAPE, "Q6_K codes must lie in 0..63");
  return make_weight_k(c, RQ_Q6_K, out, in, packed.data(), packed.size(), ds, (size_t)(out * (in / 256)) * 4, sc,
                       (size_t)(out * (in / 16)), w);
}

int rq_weight_info(rq_weight h, int* format, int64_t* out, int64_t* in, int* scale_dtype, size_t* bytes) {
  Weight* w = reinterpret_cast<Weight*>(h);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_weight(w)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_weight");
  if (format) *format = w->format;
  if (out) *out = w->out;
  if (in) *in = w->in;
  if (scale_dtype) *scale_dtype = w->scale_dtype;
  if (bytes) *bytes = w->bytes;
  return RQ_OK;
}

int rq_weight_device_ptrs(rq_weight h, const void** qdata, const void** scales) {
  Weight* w = reinterpret_cast<Weight*>(h);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_weight(w)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_weight");
  if (qdata) *qdata = w->q;
  if (scales) *scales = w->scales;
  return RQ_OK;
}

static int lookup(rq_ctx h, rq_weight wh, Ctx** c, Weight* copy) {
  Ctx* cc = reinterpret_cast<Ctx*>(h);
  Weight* w = reinterpret_cast<Weight*>(wh);
  std::lock_guard<std::mutex> lk(g_mu);
  if (!live_ctx(cc)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_ctx");
  if (!live_weight(w)) return fail(RQ_ERR_HANDLE, "unknown or destroyed rq_weight");
  if (w->device != cc->device) return fail(RQ_ERR_HANDLE, "weight lives on another device");
  *c = cc;
  *copy = *w;
  return RQ_OK;
}

}  // extern "C"

namespace rq {

// rq_qmatmul / rq_qmatmul_fused; ops == nullptr is the plain product.
// The fixed device scratch of one rq_qmatmul_noalloc call: regions are taken
// from `base` in order, 256-byte aligned, up to `cap` bytes.
struct FixedScratch {
  uint8_t* base;
  size_t cap;
  size_t used;
};

static int run_matmul(Ctx* c, const Weight& w, const DecodePlan& plan, const void* x, int x_dtype, void* y,
                      int y_dtype, int64_t m, const DecodeOps& dops, hipStream_t stream,
                      FixedScratch* fixed = nullptr);

// A scratch region of `bytes` for one call: from the fixed scratch when the
// call allocates nothing, else the stream's grow-only buffer (`which` 0: the
// packed activations, 1: the K-slices' partial sums).
static int call_scratch(Ctx* c, FixedScratch* fixed, hipStream_t stream, size_t bytes, int which, void** out) {
  if (fixed) {
    const size_t at = align256(fixed->used);
    if (bytes > fixed->cap || at > fixed->cap - bytes)
      return fail(RQ_ERR_SHAPE, "rq_qmatmul_noalloc: this call needs more than the " +
                                    std::to_string(fixed->cap >> 20) + " MiB of fixed scratch (use rq_qmatmul)");
    *out = fixed->base + at;
    fixed->used = at + bytes;
    return RQ_OK;
  }
  if (which == 0) return stream_pack(c, stream, bytes, out);
  float* p = nullptr;
  const int s = stream_split(c, stream, bytes, &p);
  *out = p;
  return s;
}

// A K-quant weight with f32 x in one call: x quantized to q8_K in scratch,
// then the K-quant GEMV -- rq_quantize_act_q8k + rq_qmatmul_q8k, with the
// same kernels and so the same results (QMatrix apply of the built-in :q4_K /
// :q6_K formats, raster/quant/core.clj:55-75).
static int run_kquant_matmul(Ctx* c, const Weight& w, const float* x, void* y, int y_dtype, int64_t m,
                             hipStream_t stream, FixedScratch* fixed) {
  const int sub = w.format == RQ_Q4_K ? 32 : 16;
  const size_t xq_b = align256((size_t)m * (size_t)w.in), xs_b = align256((size_t)m * (size_t)(w.in / 256) * 4);
  const size_t bs_b = (size_t)m * (size_t)(w.in / sub) * 4;
  if (int s = set_device(c)) return s;  // before the scratch: growing it allocates on this device
  void* buf = nullptr;
  if (int s = call_scratch(c, fixed, stream, xq_b + xs_b + bs_b, 0, &buf)) return s;
  int8_t* xq = static_cast<int8_t*>(buf);
  float* xs = reinterpret_cast<float*>(static_cast<uint8_t*>(buf) + xq_b);
  int32_t* bs = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(buf) + xq_b + xs_b);
  hipError_t e = launch_quantize_act_q8k(x, m, w.in, sub, xq, xs, bs, stream);
  if (e != hipSuccess) return hip_fail(e, "quantizer launch");
  const EvSet ev = fixed ? EvSet{} : timing_set(c, stream);
  if (ev.n) (void)hipEventRecord(ev.e[0], stream);
  e = launch_kquant_gemv(w, xq, xs, bs, y, y_dtype, m, c->cu_count, stream);
  if (ev.n && e == hipSuccess) (void)hipEventRecord(ev.e[1], stream);
  timing_done(c, ev, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "K-quant GEMV launch");
  return RQ_OK;
}

static bool kquant(const Weight& w) { return w.format == RQ_Q4_K || w.format == RQ_Q6_K; }
static const char* kKquantMsg = "K-quant weights take q8_K activations: use rq_qmatmul_q8k";
static const char* kKquantX = "K-quant weights take f32 x here (quantized to q8_K in the call), or use rq_qmatmul_q8k";

static int qmatmul_impl(rq_ctx h, rq_weight wh, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
                        const rq_fused_ops* ops, void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (kquant(w) && ops) return fail(RQ_ERR_DTYPE, "fused options need a Q8_0 or Q4_0 weight");
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  if (m > (int64_t)1 << 24) return fail(RQ_ERR_SHAPE, "m too large");
  if (!x || !y) return fail(RQ_ERR_NULL, "x or y is NULL");
  if (x_dtype != RQ_F32 && x_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "x must be f32 or bf16");
  if (y_dtype != RQ_F32 && y_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "y must be f32 or bf16");
  if (((uintptr_t)x & 15) != 0) return fail(RQ_ERR_SHAPE, "x must be 16-byte aligned");
  if (((uintptr_t)y & (y_dtype == RQ_F32 ? 3 : 1)) != 0) return fail(RQ_ERR_SHAPE, "y misaligned");
  if (kquant(w)) {
    if (x_dtype != RQ_F32) return fail(RQ_ERR_DTYPE, kKquantX);
    return run_kquant_matmul(c, w, static_cast<const float*>(x), y, y_dtype, m, (hipStream_t)stream, nullptr);
  }
  const DecodePlan plan = plan_decode(m, w.in, w.npad, c->cu_count);
  DecodeOps dops = {nullptr, 0.0f, nullptr, 0};
  if (ops) {
    if (!plan.ok) return fail(RQ_ERR_SHAPE, "fused options need the decode kernel: m <= 16");
    if (ops->norm_gain && ((uintptr_t)ops->norm_gain & 15) != 0)
      return fail(RQ_ERR_SHAPE, "norm_gain must be 16-byte aligned");
    if (ops->norm_gain && !(ops->norm_eps >= 0.0f)) return fail(RQ_ERR_SHAPE, "norm_eps must be >= 0");
    if (ops->swiglu && (w.out % 2) != 0) return fail(RQ_ERR_SHAPE, "swiglu needs an even number of rows");
    if (ops->swiglu && ops->residual) return fail(RQ_ERR_SHAPE, "swiglu and residual cannot be combined");
    if (ops->residual && ((uintptr_t)ops->residual & (y_dtype == RQ_F32 ? 3 : 1)) != 0)
      return fail(RQ_ERR_SHAPE, "residual misaligned");
    dops.norm_gain = ops->norm_gain;
    dops.norm_eps = ops->norm_eps;
    dops.residual = ops->residual;
    dops.swiglu = ops->swiglu ? 1 : 0;
    dops.act_i8 = ops->act_i8 ? 1 : 0;
  }
  return run_matmul(c, w, plan, x, x_dtype, y, y_dtype, m, dops, (hipStream_t)stream);
}

// Launches the matmul of a validated call: for m <= 16 the int8 decode kernel
// (for m = 1 with Q4_0 weights the sdot4 GEMV instead, unless a norm,
// residual or SwiGLU is fused; without fused options and with f32 / bf16 x,
// the MFMA decode kernel where plan_gemv_mf takes the shape: Q4_0 at
// 5 <= m <= 16, Q8_0 at 9 <= m <= 16 up to 32 Mi weight elements), else the
// GEMM for the activation dtype; per-stream scratch and kernel timing around
// it.
static int run_matmul(Ctx* c, const Weight& w, const DecodePlan& plan, const void* x, int x_dtype, void* y,
                      int y_dtype, int64_t m, const DecodeOps& dops, hipStream_t stream, FixedScratch* fixed) {
  if (int s = set_device(c)) return s;
  MatmulArgs a;
  a.q = w.q;
  a.scales = w.scales;
  a.scales_rb = w.scales_rb;
  a.scale_dtype = w.scale_dtype;
  a.format = w.format;
  a.x = x;
  a.x_dtype = x_dtype;
  a.y = y;
  a.y_dtype = y_dtype;
  a.m = m;
  a.k = w.in;
  a.n = w.out;
  a.npad = w.npad;
  a.stream = stream;
  a.scratch = nullptr;
  a.part = nullptr;
  a.ops = dops;
  const bool plain = !dops.norm_gain && !dops.residual && !dops.swiglu && !dops.act_i8;
  const MfPlan mf = plain && plan.ok ? plan_gemv_mf(m, w.in, w.npad, x_dtype, w.format, c->cu_count) : MfPlan{};
  // the m = 1 GEMV also quantizes to int8 blocks itself (act_i8)
  const bool plain_g1 = !dops.norm_gain && !dops.residual && !dops.swiglu;
  const G1Plan g1 = plain_g1 && plan.ok ? plan_gemv1(m, w.in, w.npad, x_dtype, w.format, c->cu_count) : G1Plan{};
  // bf16 x past the decode and small-m kernels: the 256 x 192 GEMM where its
  // plan takes the shape
  const WidePlan wide = !plan.ok && x_dtype == RQ_BF16 && !gemm_sm_takes(w.format, m, w.in)
                            ? plan_gemm_wide(m, w.in, w.npad, c->cu_count)
                            : WidePlan{};
  void* part = nullptr;
  if (g1.ok) {
    // the m = 1 GEMV uses no scratch
  } else if (mf.ok) {
    if (mf.ks > 1) {
      if (int s = call_scratch(c, fixed, a.stream, (size_t)mf.ks * (size_t)m * (size_t)w.out * 4, 1, &part))
        return s;
    }
  } else if (plan.ok && plan.ksplit > 1) {
    if (int s = call_scratch(c, fixed, a.stream, plan.part_bytes, 1, &part)) return s;
  } else if (!plan.ok && x_dtype == RQ_BF16 && wide.ok) {
    // the 32x32x16 operand copy of x: ceil(m/32)*32 rows
    if (int s = call_scratch(c, fixed, a.stream, pack_x32_bytes(m, w.in), 0, &a.scratch)) return s;
  } else if (!plan.ok && x_dtype == RQ_BF16 && gemm_sm_takes(w.format, m, w.in)) {
    // the weight-stream GEMM reads x as it is; K-slices' partial sums
    a.slices = gemm_sm_slices(w.format, m, w.in, w.npad, c->cu_count);
    if (a.slices > 1) {
      if (int s = call_scratch(c, fixed, a.stream, (size_t)a.slices * (size_t)m * (size_t)w.out * 4, 1, &part))
        return s;
    }
  } else if (!plan.ok && x_dtype == RQ_BF16) {
    // fragment-major copy of the activations: ceil(m/16)*16 rows (16x16x32
    // operands), or ceil(m/32)*32 rows for the 32x32x16 K-pair kernel
    const size_t bytes = std::max((size_t)((m + 15) / 16 * 16) * (size_t)w.in * 2, pack_x32_bytes(m, w.in));
    if (int s = call_scratch(c, fixed, a.stream, bytes, 0, &a.scratch)) return s;
  } else if (!plan.ok && x_dtype == kXtI8) {
    // fragment-major int8 activations with their scales and sums: 640 B per
    // 16-row tile and 32-block
    const size_t bytes = (size_t)((m + 15) / 16) * (size_t)(w.in / 32) * 640;
    if (int s = call_scratch(c, fixed, a.stream, bytes, 0, &a.scratch)) return s;
  }
  a.part = static_cast<float*>(part);
  // no timing events for calls that allocate nothing (creating one allocates);
  // calls whose partial sums a second kernel adds time both kernels
  const bool two = (mf.ok && mf.ks > 1) || (!mf.ok && !g1.ok && plan.ok && plan.ksplit > 1) || a.slices > 1;
  const EvSet ev = fixed ? EvSet{} : timing_set(c, a.stream, two);
  a.ev_main[0] = ev.e[0];
  a.ev_main[1] = ev.e[1];
  if (ev.n == 4) {
    a.ev_aux[0] = ev.e[2];
    a.ev_aux[1] = ev.e[3];
  }
  hipError_t e = g1.ok                ? launch_gemv1(a, g1)
                 : mf.ok              ? launch_gemv_mf(a, mf)
                 : plan.ok            ? launch_gemv(a, plan)
                 : x_dtype == kXtI8   ? launch_gemm_i8(a, c->cu_count)
                 : x_dtype == RQ_BF16 ? (gemm_sm_takes(w.format, m, w.in) ? launch_gemm_sm(a, a.slices)
                                         : wide.ok ? launch_gemm_wide(a, wide)
                                                 : launch_gemm_bf16(a, c->cu_count))
                                      : launch_gemm(a, c->cu_count);
  timing_done(c, ev, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "kernel launch");
  return RQ_OK;
}

}  // namespace rq

extern "C" {

int rq_qmatmul(rq_ctx h, rq_weight wh, const void* x, int x_dtype, void* y, int y_dtype, int64_t m, void* stream) {
  return qmatmul_impl(h, wh, x, x_dtype, y, y_dtype, m, nullptr, stream);
}

int rq_qmatmul_noalloc(rq_ctx h, rq_weight wh, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
                       void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  if (m > (int64_t)1 << 24) return fail(RQ_ERR_SHAPE, "m too large");
  if (!x || !y) return fail(RQ_ERR_NULL, "x or y is NULL");
  if (x_dtype != RQ_F32 && x_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "x must be f32 or bf16");
  if (y_dtype != RQ_F32 && y_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "y must be f32 or bf16");
  if (((uintptr_t)x & 15) != 0) return fail(RQ_ERR_SHAPE, "x must be 16-byte aligned");
  if (((uintptr_t)y & (y_dtype == RQ_F32 ? 3 : 1)) != 0) return fail(RQ_ERR_SHAPE, "y misaligned");
  if (kquant(w) && x_dtype != RQ_F32) return fail(RQ_ERR_DTYPE, kKquantX);
  void* ptr;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    ptr = g_scratch_ptr[c->device];  // set when the context was created
  }
  if (!ptr) return fail(RQ_ERR_HIP, "no device address for the fixed scratch of this device");
  FixedScratch fs = {static_cast<uint8_t*>(ptr), kNoAllocScratchBytes, 0};
  if (kquant(w))
    return run_kquant_matmul(c, w, static_cast<const float*>(x), y, y_dtype, m, (hipStream_t)stream, &fs);
  const DecodePlan plan = plan_decode(m, w.in, w.npad, c->cu_count);
  const DecodeOps dops = {nullptr, 0.0f, nullptr, 0, 0, nullptr, nullptr};
  return run_matmul(c, w, plan, x, x_dtype, y, y_dtype, m, dops, (hipStream_t)stream, &fs);
}

int rq_qmatmul_fused(rq_ctx h, rq_weight wh, const void* x, int x_dtype, void* y, int y_dtype, int64_t m,
                     const rq_fused_ops* ops, void* stream) {
  if (!ops) return fail(RQ_ERR_NULL, "ops is NULL");
  return qmatmul_impl(h, wh, x, x_dtype, y, y_dtype, m, ops, stream);
}

int rq_quantize_act_i8(rq_ctx h, const float* x, int64_t m, int64_t in, int8_t* xq, float* xs, int32_t* xsum,
                       void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (m < 0 || in < 0) return fail(RQ_ERR_SHAPE, "negative dimension");
  if (in % 32 != 0) return fail(RQ_ERR_SHAPE, "in must be a multiple of 32");
  if (m == 0 || in == 0) return RQ_OK;
  if (m > ((int64_t)1 << 40) / in) return fail(RQ_ERR_SHAPE, "m * in too large");
  if (!x || !xq || !xs) return fail(RQ_ERR_NULL, "x, xq or xs is NULL");
  if (((uintptr_t)x & 15) != 0) return fail(RQ_ERR_SHAPE, "x must be 16-byte aligned");
  if (((uintptr_t)xq & 3) != 0 || ((uintptr_t)xs & 3) != 0 || ((uintptr_t)xsum & 3) != 0)
    return fail(RQ_ERR_SHAPE, "xq, xs and xsum must be 4-byte aligned");
  if (int s = set_device(c)) return s;
  hipError_t e = launch_quantize_act_i8(x, m, in, xq, xs, xsum, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantizer launch");
  return RQ_OK;
}

int rq_qmatmul_i8(rq_ctx h, rq_weight wh, const int8_t* xq, const float* xs, const int32_t* xsum, void* y,
                  int y_dtype, int64_t m, void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (kquant(w)) return fail(RQ_ERR_DTYPE, kKquantMsg);
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  if (m > (int64_t)1 << 24) return fail(RQ_ERR_SHAPE, "m too large");
  if (!xq || !xs || !y) return fail(RQ_ERR_NULL, "xq, xs or y is NULL");
  if (w.format == RQ_Q4_0 && !xsum) return fail(RQ_ERR_NULL, "Q4_0 needs xsum (the zero-point fold)");
  if (y_dtype != RQ_F32 && y_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "y must be f32 or bf16");
  if (((uintptr_t)xq & 15) != 0) return fail(RQ_ERR_SHAPE, "xq must be 16-byte aligned");
  if (((uintptr_t)xs & 3) != 0 || ((uintptr_t)xsum & 3) != 0) return fail(RQ_ERR_SHAPE, "xs / xsum misaligned");
  if (((uintptr_t)y & (y_dtype == RQ_F32 ? 3 : 1)) != 0) return fail(RQ_ERR_SHAPE, "y misaligned");
  const DecodePlan plan = plan_decode(m, w.in, w.npad, c->cu_count);
  DecodeOps dops{};
  dops.act_scale = xs;
  dops.act_sum = w.format == RQ_Q4_0 ? xsum : nullptr;
  return run_matmul(c, w, plan, xq, kXtI8, y, y_dtype, m, dops, (hipStream_t)stream);
}

int rq_quantize_act_q8k(rq_ctx h, const float* x, int64_t m, int64_t in, int sub, int8_t* xq, float* xs,
                        int32_t* bsums, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (m < 0 || in < 0) return fail(RQ_ERR_SHAPE, "negative dimension");
  if (in % 256 != 0) return fail(RQ_ERR_SHAPE, "in must be a multiple of 256");
  if (sub != 32 && sub != 16) return fail(RQ_ERR_SHAPE, "sub must be 32 (Q4_K) or 16 (Q6_K)");
  if (m == 0 || in == 0) return RQ_OK;
  if (m > ((int64_t)1 << 40) / in) return fail(RQ_ERR_SHAPE, "m * in too large");
  if (!x || !xq || !xs || !bsums) return fail(RQ_ERR_NULL, "NULL argument");
  if (((uintptr_t)x & 15) != 0) return fail(RQ_ERR_SHAPE, "x must be 16-byte aligned");
  if (((uintptr_t)xq & 3) != 0 || ((uintptr_t)xs & 3) != 0 || ((uintptr_t)bsums & 3) != 0)
    return fail(RQ_ERR_SHAPE, "xq, xs and bsums must be 4-byte aligned");
  if (int s = set_device(c)) return s;
  hipError_t e = launch_quantize_act_q8k(x, m, in, sub, xq, xs, bsums, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantizer launch");
  return RQ_OK;
}

int rq_qmatmul_q8k(rq_ctx h, rq_weight wh, const int8_t* xq, const float* xs, const int32_t* bsums, void* y,
                   int y_dtype, int64_t m, void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (!kquant(w)) return fail(RQ_ERR_DTYPE, "rq_qmatmul_q8k needs a Q4_K or Q6_K weight");
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  if (m > (int64_t)1 << 24) return fail(RQ_ERR_SHAPE, "m too large");
  if (!xq || !xs || !bsums || !y) return fail(RQ_ERR_NULL, "NULL argument");
  if (y_dtype != RQ_F32 && y_dtype != RQ_BF16) return fail(RQ_ERR_DTYPE, "y must be f32 or bf16");
  if (((uintptr_t)xq & 15) != 0) return fail(RQ_ERR_SHAPE, "xq must be 16-byte aligned");
  if (((uintptr_t)xs & 3) != 0 || ((uintptr_t)bsums & 3) != 0) return fail(RQ_ERR_SHAPE, "xs / bsums misaligned");
  if (((uintptr_t)y & (y_dtype == RQ_F32 ? 3 : 1)) != 0) return fail(RQ_ERR_SHAPE, "y misaligned");
  if (int s = set_device(c)) return s;
  const EvSet ev = timing_set(c, (hipStream_t)stream);
  if (ev.n) (void)hipEventRecord(ev.e[0], (hipStream_t)stream);
  hipError_t e = launch_kquant_gemv(w, xq, xs, bsums, y, y_dtype, m, c->cu_count, (hipStream_t)stream);
  if (ev.n && e == hipSuccess) (void)hipEventRecord(ev.e[1], (hipStream_t)stream);
  timing_done(c, ev, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "K-quant GEMV launch");
  return RQ_OK;
}

int rq_decode_attention(rq_ctx h, const float* q, const float* k, const float* v, float* kcache, float* vcache,
                        int64_t pos, int64_t n_q, int64_t n_kv, int64_t head_dim, double theta, double scale,
                        float* out, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!q || !k || !v || !kcache || !vcache || !out) return fail(RQ_ERR_NULL, "NULL argument");
  if (pos < 0 || n_q <= 0 || n_kv <= 0 || head_dim <= 0) return fail(RQ_ERR_SHAPE, "negative or zero dimension");
  if (n_q % n_kv != 0) return fail(RQ_ERR_SHAPE, "n_q must be a multiple of n_kv");
  if (head_dim % 2 != 0) return fail(RQ_ERR_SHAPE, "head_dim must be even");
  if (n_q > 65535 || head_dim > 65536 || pos > INT32_MAX - 1) return fail(RQ_ERR_SHAPE, "dimension too large");
  if (decode_attention_lds(pos, head_dim) > 163840)
    return fail(RQ_ERR_SHAPE, "cache longer than one workgroup's LDS holds (head_dim not a multiple of 4 "
                              "or above 512: about 40K positions)");
  if (!(theta > 0.0)) return fail(RQ_ERR_SHAPE, "theta must be positive");
  if (int s = set_device(c)) return s;
  const AttnSplit sp = plan_decode_attention(pos, n_q, n_kv, head_dim, c->cu_count);
  void* scratch_buf = nullptr;
  if (sp.nsplit > 1)
    if (int s = stream_attn(c, (hipStream_t)stream, sp.scratch_bytes, &scratch_buf)) return s;
  hipError_t e = launch_decode_attention(q, k, v, kcache, vcache, pos, n_q, n_kv, head_dim, theta, scale, out, sp,
                                         scratch_buf, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "attention launch");
  return RQ_OK;
}

int rq_dequant(rq_ctx h, rq_weight wh, float* w_out, void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (!w_out) return fail(RQ_ERR_NULL, "w_out is NULL");
  if (((uintptr_t)w_out & 15) != 0) return fail(RQ_ERR_SHAPE, "w_out must be 16-byte aligned");
  if (int s = set_device(c)) return s;
  hipError_t e = kquant(w) ? launch_kquant_dequant(w, w_out, (hipStream_t)stream)
                           : launch_dequant(w, w_out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dequant launch");
  return RQ_OK;
}

int rq_qlinear_q8(rq_ctx h, const float* x, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                  int64_t out, float* y) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!x || !codes || !scales || !y) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  rq_weight w = nullptr;
  if (int s = rq_weight_create_q8(h, codes, scales, out, in, &w)) return s;
  void *dx = nullptr, *dy = nullptr;
  int s = rq_buf_alloc(h, (size_t)(m * in) * 4, &dx);
  if (!s) s = rq_buf_alloc(h, (size_t)(m * out) * 4, &dy);
  if (!s) s = rq_upload(h, dx, x, (size_t)(m * in) * 4, nullptr);
  if (!s) s = rq_qmatmul(h, w, dx, RQ_F32, dy, RQ_F32, m, nullptr);
  if (!s) s = rq_download(h, y, dy, (size_t)(m * out) * 4, nullptr);
  std::string keep = s ? t_err : std::string();
  if (dx) rq_buf_free(h, dx);
  if (dy) rq_buf_free(h, dy);
  rq_weight_destroy(w);
  if (s) t_err = keep;
  return s;
}

int rq_qmatmul_dx(rq_ctx h, rq_weight wh, const float* dy, float* dx, int64_t m, void* stream) {
  Ctx* c;
  Weight w;
  if (int s = lookup(h, wh, &c, &w)) return s;
  if (kquant(w)) return fail(RQ_ERR_DTYPE, "rq_qmatmul_dx supports Q8_0 and Q4_0 weights");
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  if (m > (int64_t)1 << 24) return fail(RQ_ERR_SHAPE, "m too large");
  if (!dy || !dx) return fail(RQ_ERR_NULL, "dy or dx is NULL");
  if (((uintptr_t)dy & 3) != 0) return fail(RQ_ERR_SHAPE, "dy must be 4-byte aligned");
  if (((uintptr_t)dx & 15) != 0) return fail(RQ_ERR_SHAPE, "dx must be 16-byte aligned");
  if (int s = set_device(c)) return s;
  const hipStream_t st = (hipStream_t)stream;
  // m <= kDxFmMaxRows: f32 MFMA on the weight as stored (weight read once per
  // 16 dy rows); above it the bf16 MFMA GEMM (once per 128 rows)
  const bool mf = m > kDxFmMaxRows;
  const int slices = mf ? dx_mf_slices(m, w.in, w.npad, c->cu_count) : dx_fm_slices(m, w.in, w.npad, c->cu_count);
  float* part = nullptr;
  void* pack = nullptr;
  if (slices > 1) {
    if (int s = stream_split(c, st, (size_t)slices * (size_t)m * (size_t)w.in * 4, &part)) return s;
  }
  if (mf)
    if (int s = stream_pack(c, st, dx_mf_pack_bytes(m, w.npad), &pack)) return s;
  const EvSet ev = timing_set(c, st);
  if (ev.n) (void)hipEventRecord(ev.e[0], st);
  hipError_t e = mf ? launch_dx_mf(w, dy, dx, m, pack, part, slices, st) : launch_dx_fm(w, dy, dx, m, part, slices, st);
  if (ev.n && e == hipSuccess) (void)hipEventRecord(ev.e[1], st);
  timing_done(c, ev, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "dx launch");
  return RQ_OK;
}

int rq_nextpad(int64_t in, int64_t* inp) {
  if (!inp) return fail(RQ_ERR_NULL, "inp is NULL");
  if (in <= 0 || in > ((int64_t)1 << 40)) return fail(RQ_ERR_SHAPE, "in must be in 1 .. 2^40");
  *inp = (in + 255) / 256 * 256;
  return RQ_OK;
}

int rq_q8_quantize(rq_ctx h, const float* W, int64_t out, int64_t in, int8_t* codes, float* scales, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!W || !codes || !scales) return fail(RQ_ERR_NULL, "W, codes or scales is NULL");
  if (int s = check_shape(out, in)) return s;
  if (((uintptr_t)W & 15) != 0) return fail(RQ_ERR_SHAPE, "W must be 16-byte aligned");
  if (((uintptr_t)codes & 3) != 0 || ((uintptr_t)scales & 3) != 0)
    return fail(RQ_ERR_SHAPE, "codes and scales must be 4-byte aligned");
  if (int s = set_device(c)) return s;
  // q8-quantize's per-block math is quantize-act-i8's (d = max|w| / 127 in
  // double, Math/round, clamp to +-127): the same kernel over out rows of in
  hipError_t e = launch_quantize_act_i8(W, out, in, codes, scales, nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantizer launch");
  return RQ_OK;
}

int rq_q4k_of(rq_ctx h, const float* W, int64_t out, int64_t in, uint8_t* wq, float* da, float* db, uint8_t* aq,
              int8_t* bq, int64_t* inp, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!W || !wq || !da || !db || !aq || !bq || !inp) return fail(RQ_ERR_NULL, "NULL argument");
  if (out <= 0 || in <= 0) return fail(RQ_ERR_SHAPE, "out and in must be positive");
  if (in > (int64_t)1 << 30 || out > (int64_t)1 << 30) return fail(RQ_ERR_SHAPE, "dimension too large");
  if (((uintptr_t)wq & 15) != 0 || ((uintptr_t)da & 3) != 0 || ((uintptr_t)db & 3) != 0)
    return fail(RQ_ERR_SHAPE, "wq must be 16-byte aligned, da and db 4-byte aligned");
  if (int s = rq_nextpad(in, inp)) return s;
  if (int s = set_device(c)) return s;
  hipError_t e = launch_q4k_encode(W, out, in, *inp, wq, da, db, aq, bq, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "encoder launch");
  return RQ_OK;
}

int rq_quantize_weight_q6k(rq_ctx h, const float* W, int64_t out, int64_t in, uint8_t* wq, int8_t* sc, float* ds,
                           void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!W || !wq || !sc || !ds) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  if (in % 256 != 0) return fail(RQ_ERR_SHAPE, "quantize-weight-q6k needs in % 256 == 0 (super-blocks of 256)");
  if (((uintptr_t)W & 15) != 0 || ((uintptr_t)wq & 15) != 0 || ((uintptr_t)ds & 3) != 0)
    return fail(RQ_ERR_SHAPE, "W and wq must be 16-byte aligned, ds 4-byte aligned");
  if (int s = set_device(c)) return s;
  hipError_t e = launch_q6k_encode(W, out, in, wq, sc, ds, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "encoder launch");
  return RQ_OK;
}

int rq_qlinear_i8(rq_ctx h, const float* x, const uint8_t* wqi, const float* wsi, int nibble, float* y, int64_t in,
                  int64_t out) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!x || !wqi || !wsi || !y) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  if (out % 8 != 0) return fail(RQ_ERR_SHAPE, "x8 layout needs out % 8 == 0");
  rq_weight w = nullptr;
  if (int s = rq_weight_create_x8(h, wqi, wsi, nibble ? 1 : 0, out, in, &w)) return s;
  void *dx = nullptr, *dy = nullptr;
  int s = rq_buf_alloc(h, (size_t)in * 4, &dx);
  if (!s) s = rq_buf_alloc(h, (size_t)out * 4, &dy);
  if (!s) s = rq_upload(h, dx, x, (size_t)in * 4, nullptr);
  rq_fused_ops ops = {nullptr, 0.0f, nullptr, 0, 1};  // act_i8: quantize-act-i8 in the kernel
  if (!s) s = rq_qmatmul_fused(h, w, dx, RQ_F32, dy, RQ_F32, 1, &ops, nullptr);
  if (!s) s = rq_download(h, y, dy, (size_t)out * 4, nullptr);
  std::string keep = s ? t_err : std::string();
  if (dx) rq_buf_free(h, dx);
  if (dy) rq_buf_free(h, dy);
  rq_weight_destroy(w);
  if (s) t_err = keep;
  return s;
}

int rq_i8gemv_dp4a(rq_ctx h, const int32_t* wp, const int32_t* xp, float* y, int64_t kw, int64_t out,
                   void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (kw < 0 || out < 0) return fail(RQ_ERR_SHAPE, "negative dimension");
  if (out == 0) return RQ_OK;
  if (!y || (kw > 0 && (!wp || !xp))) return fail(RQ_ERR_NULL, "wp, xp or y is NULL");
  if (kw > ((int64_t)1 << 20)) return fail(RQ_ERR_SHAPE, "kw above 2^20 words (the lanes' int32 partial sums)");
  if (out > ((int64_t)1 << 40) / std::max<int64_t>(kw, 1)) return fail(RQ_ERR_SHAPE, "out * kw too large");
  if ((((uintptr_t)wp | (uintptr_t)xp) & 3) != 0 || ((uintptr_t)y & 3) != 0)
    return fail(RQ_ERR_SHAPE, "wp, xp and y must be 4-byte aligned");
  if (int s = set_device(c)) return s;
  const hipError_t e = launch_i8gemv_dp4a(wp, xp, y, kw, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "i8gemv launch");
  return RQ_OK;
}

int rq_stream_read(rq_ctx h, const void* src, size_t bytes, int wg_per_cu, uint32_t* sink, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!src || !sink) return fail(RQ_ERR_NULL, "src or sink is NULL");
  if (bytes == 0 || bytes % 16 != 0 || ((uintptr_t)src & 15) != 0)
    return fail(RQ_ERR_SHAPE, "bytes must be a positive multiple of 16 and src 16-byte aligned");
  if (wg_per_cu < 1 || wg_per_cu > 16) return fail(RQ_ERR_SHAPE, "wg_per_cu must be 1 .. 16");
  if (int s = set_device(c)) return s;
  const EvSet ev = timing_set(c, (hipStream_t)stream);
  if (ev.n) (void)hipEventRecord(ev.e[0], (hipStream_t)stream);
  hipError_t e = launch_stream_read(src, bytes, c->cu_count * wg_per_cu, sink, (hipStream_t)stream);
  if (ev.n && e == hipSuccess) (void)hipEventRecord(ev.e[1], (hipStream_t)stream);
  timing_done(c, ev, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "stream read launch");
  return RQ_OK;
}

int rq_qlinear_q8_dx(rq_ctx h, const float* dy, const int8_t* codes, const float* scales, int64_t m, int64_t in,
                     int64_t out, float* dx) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (!dy || !codes || !scales || !dx) return fail(RQ_ERR_NULL, "NULL argument");
  if (int s = check_shape(out, in)) return s;
  if (m < 0) return fail(RQ_ERR_SHAPE, "m < 0");
  if (m == 0) return RQ_OK;
  rq_weight w = nullptr;
  if (int s = rq_weight_create_q8(h, codes, scales, out, in, &w)) return s;
  void *ddy = nullptr, *ddx = nullptr;
  int s = rq_buf_alloc(h, (size_t)(m * out) * 4, &ddy);
  if (!s) s = rq_buf_alloc(h, (size_t)(m * in) * 4, &ddx);
  if (!s) s = rq_upload(h, ddy, dy, (size_t)(m * out) * 4, nullptr);
  if (!s) s = rq_qmatmul_dx(h, w, static_cast<const float*>(ddy), static_cast<float*>(ddx), m, nullptr);
  if (!s) s = rq_download(h, dx, ddx, (size_t)(m * in) * 4, nullptr);
  std::string keep = s ? t_err : std::string();
  if (ddy) rq_buf_free(h, ddy);
  if (ddx) rq_buf_free(h, ddx);
  rq_weight_destroy(w);
  if (s) t_err = keep;
  return s;
}

}  // extern "C"

// ---- dense f32 GEMM (Raster's blas/dgemm! float arms and nn/linear!)

namespace rq {

// C[m x n] = alpha op(A) op(B) + beta C through the context's rocBLAS handle.
// Like Raster's arms (blas.clj:301, 318, 334), a call with m, n or k not
// positive does nothing.
static int dense_call(rq_ctx h, int trans_a, int trans_b, const float* a, const float* b, float* c, int64_t m,
                      int64_t k, int64_t n, float alpha, float beta, void* stream) {
  Ctx* ctx = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(ctx)) return s;
  if (m <= 0 || n <= 0 || k <= 0) return RQ_OK;
  if (!a || !b || !c) return fail(RQ_ERR_NULL, "NULL argument");
  if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX) return fail(RQ_ERR_SHAPE, "dimension above 2^31 - 1");
  if (int s = set_device(ctx)) return s;
  std::lock_guard<std::mutex> lk(ctx->blas_mu);
  if (!ctx->blas) {
    if (capturing((hipStream_t)stream))
      return fail(RQ_ERR_SHAPE, "the dense GEMM's library handle is created on the first call, which cannot be "
                                "under HIP graph capture: make one call on any stream before capturing");
    void* hb = nullptr;
    if (int st = dense_create(&hb))
      return fail(RQ_ERR_HIP, std::string("rocblas_create_handle: ") + dense_status_string(st));
    ctx->blas = hb;
  }
  if (int st = dense_sgemm(ctx->blas, (hipStream_t)stream, trans_a, trans_b, m, n, k, alpha, a, b, beta, c))
    return fail(RQ_ERR_HIP, std::string("rocblas_sgemm: ") + dense_status_string(st));
  return RQ_OK;
}

}  // namespace rq

extern "C" {

int rq_sgemm(rq_ctx h, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
             float beta, void* stream) {
  return dense_call(h, 0, 0, a, b, c, m, k, n, alpha, beta, stream);
}

int rq_sgemm_tn(rq_ctx h, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
                float beta, void* stream) {
  return dense_call(h, 1, 0, a, b, c, m, k, n, alpha, beta, stream);
}

int rq_sgemm_nt(rq_ctx h, const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n, float alpha,
                float beta, void* stream) {
  return dense_call(h, 0, 1, a, b, c, m, k, n, alpha, beta, stream);
}

int rq_linear(rq_ctx h, const float* x, const float* w, const float* b, float* y, int64_t batch, int64_t in_f,
              int64_t out_f, void* stream) {
  Ctx* c = reinterpret_cast<Ctx*>(h);
  if (int s = check_ctx(c)) return s;
  if (batch <= 0 || out_f <= 0) return RQ_OK;
  if (!b || !y || (in_f > 0 && (!x || !w))) return fail(RQ_ERR_NULL, "NULL argument");
  if (batch > INT32_MAX || out_f > INT32_MAX || in_f > INT32_MAX) return fail(RQ_ERR_SHAPE, "dimension above 2^31 - 1");
  if (int s = set_device(c)) return s;
  // y = b in every row, then y = 1 x W^T + 1 y (nn.clj:166-173)
  if (hipError_t e = launch_bias_rows(b, y, batch, out_f, (hipStream_t)stream)) return hip_fail(e, "bias launch");
  return dense_call(h, 0, 1, x, w, y, batch, in_f, out_f, 1.0f, 1.0f, stream);
}

}  // extern "C"
