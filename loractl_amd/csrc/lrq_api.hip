// The C ABI of libloractl_rocm.so (include/loractl_rocm.h): context, stream,
// workspace, argument validation, per-kernel timing, and the call sequences
// of the fused forward and backward.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <functional>
#include <mutex>
#include <new>
#include <vector>

#include "lrq_kernels.h"

void set_num_cus(int n);

struct lrq_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  char* ws_alloc = nullptr;   // the allocation: arrival counters, then the workspace
  uint32_t* cnt = nullptr;    // LRQ_CNT_WORDS arrival counters of the few-token kernels
  char* ws = nullptr;         // ws_alloc + LRQ_CNT_BYTES
  size_t ws_bytes = 0;
  // set once a call has run while the stream was being captured: from then
  // on a growing workspace keeps the old allocations (a captured graph may
  // still point at them) until lrq_destroy
  bool captured = false;
  std::vector<char*> retired;
  char err[512] = {0};
  bool prof = false;
  struct Rec {
    int kid;
    hipEvent_t a, b;
  };
  std::vector<Rec> pending;
  std::vector<hipEvent_t> pool;
  double total_ms[KID_COUNT] = {0};
  int64_t launches[KID_COUNT] = {0};
  // the last launch of each hot kernel with its arguments, for
  // lrq_profile_relaunch (timing one kernel alone)
  std::function<hipError_t()> last[KID_COUNT];
};

// The workspace of lrq_lora_fwd_noalloc: a file-scope device array, one
// copy per GPU, held until the process ends. In host code its name is not a
// device address; lrq_create looks up each device's copy once
// (hipGetSymbolAddress, with that device current) and every later use goes
// through that pointer.
static __device__ __align__(256) char scratch[LRQ_NOALLOC_SCRATCH_BYTES];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static char* g_scratch[kMaxDevices] = {};

// Look up the current device's copy of `scratch` (once per device).
static int init_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return LRQ_EUNSUPPORTED;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch[device]) return LRQ_OK;
  void* p = nullptr;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LRQ_EHIP;
  g_scratch[device] = static_cast<char*>(p);
  return LRQ_OK;
}

namespace {

const char* kNames[KID_COUNT] = {"quantize_int4", "quantize_fp8", "dequant", "fwd_main", "bwd_dx", "lora_t",
                                 "lora_u",        "lora_da",      "lora_db", "block",    "lora_dadb",
                                 "quantize_int8"};

int fail(lrq_ctx* c, int code, const char* fmt, ...) {
  if (c) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(c->err, sizeof(c->err), fmt, ap);
    va_end(ap);
  }
  return code;
}

int hip_fail(lrq_ctx* c, hipError_t e, const char* what) {
  return fail(c, LRQ_EHIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

hipEvent_t take_event(lrq_ctx* c) {
  if (!c->pool.empty()) {
    hipEvent_t e = c->pool.back();
    c->pool.pop_back();
    return e;
  }
  // timing only: no system-scope fence (a cache write-back per marker
  // would be timed with the kernel it brackets)
  hipEvent_t e = nullptr;
  if (hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) return nullptr;
  return e;
}

// Run one launcher; when profiling, bracket it with events on the stream.
template <class F>
int run(lrq_ctx* c, int kid, const char* what, F&& f) {
  hipEvent_t a = nullptr, b = nullptr;
  if (c->prof) {
    a = take_event(c);
    if (a) (void)hipEventRecord(a, c->stream);
  }
  hipError_t e = f();
  if (e != hipSuccess) return hip_fail(c, e, what);
  if (c->prof && a) {
    b = take_event(c);
    if (b) {
      (void)hipEventRecord(b, c->stream);
      c->pending.push_back({kid, a, b});
    } else {
      c->pool.push_back(a);
    }
  }
  return LRQ_OK;
}

// A launch of the fused calls: run it, and keep it (arguments by value) so
// that lrq_profile_relaunch can repeat exactly this launch.
template <class F>
int run_hot(lrq_ctx* c, int kid, const char* what, F f) {
  const int rc = run(c, kid, what, f);
  if (rc == LRQ_OK) c->last[kid] = f;
  return rc;
}

// A forward (backward) call forgets the recorded launches of every kernel
// its pass may launch, so that lrq_profile_relaunch repeats only launches of
// the pass's latest call: a kernel that call did not launch (the shape took
// another path) has none to repeat, rather than one whose buffers may be
// gone.
void forget_pass(lrq_ctx* c, bool bwd) {
  static const int fwd_k[] = {KID_FWD_MAIN, KID_LORA_T};
  static const int bwd_k[] = {KID_BWD_DX, KID_LORA_U, KID_LORA_DA, KID_LORA_DB, KID_LORA_DADB};
  if (bwd)
    for (int k : bwd_k) c->last[k] = nullptr;
  else
    for (int k : fwd_k) c->last[k] = nullptr;
}

int flush_profile(lrq_ctx* c) {
  for (auto& r : c->pending) {
    hipError_t e = hipEventSynchronize(r.b);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventSynchronize");
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) return hip_fail(c, e, "hipEventElapsedTime");
    c->total_ms[r.kid] += ms;
    c->launches[r.kid] += 1;
    c->pool.push_back(r.a);
    c->pool.push_back(r.b);
  }
  c->pending.clear();
  return LRQ_OK;
}

// Bump allocator over the context workspace (256-byte aligned slices).
struct Slab {
  char* base;
  size_t off = 0;
  template <class T>
  T* take(int64_t count) {
    T* p = reinterpret_cast<T*>(base ? base + off : nullptr);
    off += (size_t)round_up((int64_t)(count * (int64_t)sizeof(T)), 256);
    return p;
  }
};

int ensure_ws(lrq_ctx* c, size_t bytes) {
  if (c->ws && bytes <= c->ws_bytes) return LRQ_OK;
  // growing the workspace synchronizes the stream and allocates, neither of
  // which a stream under graph capture allows: refuse instead
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(c->stream, &cap);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(c, LRQ_EINVAL,
                "the workspace must grow to %zu bytes (has %zu) while the stream is being captured: call "
                "lrq_reserve for this shape before capturing",
                bytes, c->ws_bytes);
  // stream-ordered users of the old buffer must finish before it goes
  e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
  // launches kept for lrq_profile_relaunch point into the old workspace
  for (auto& f : c->last) f = nullptr;
  if (c->ws_alloc) {
    // a graph captured on this context may still replay kernels that read
    // and write the old allocation: keep it until lrq_destroy
    if (c->captured)
      c->retired.push_back(c->ws_alloc);
    else
      (void)hipFree(c->ws_alloc);
  }
  c->ws_alloc = c->ws = nullptr;
  c->cnt = nullptr;
  c->ws_bytes = 0;
  size_t want = (size_t)round_up((int64_t)(bytes > 0 ? bytes : 1), 1 << 20);
  e = hipMalloc(&c->ws_alloc, want + LRQ_CNT_BYTES);
  if (e != hipSuccess) {
    c->ws_alloc = nullptr;
    return fail(c, LRQ_ENOMEM, "workspace of %zu bytes: %s", want, hipGetErrorString(e));
  }
  // the few-token kernels' arrival counters start at zero (and each launch
  // leaves them at zero)
  e = hipMemsetAsync(c->ws_alloc, 0, LRQ_CNT_BYTES, c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "hipMemsetAsync");
  c->cnt = reinterpret_cast<uint32_t*>(c->ws_alloc);
  c->ws = c->ws_alloc + LRQ_CNT_BYTES;
  c->ws_bytes = want;
  return LRQ_OK;
}

// Workspace layout of the fused calls (sizes only when base == nullptr): t
// and u padded to rp columns (the GEMM epilogue operands) and the f32
// partials of the LoRA reductions (t or u; dA and dB side by side).
// f32 partials of the fused GEMMs when they split the depth (few output
// tiles): the larger of the forward's and the backward's
int64_t gemm_part_floats(int64_t m, int64_t n, int64_t k) {
  return std::max(gemm_split_floats(m, n, k), gemm_split_floats(m, k, n));
}

// LoRA workspace: t and u padded to rp columns, the weight-side factor rows
// of the fused GEMM's LoRA step (B^T [n, rp] forward, A [k, rp] backward),
// the side kernels' f32 partials and the fused GEMMs' split partials.
struct LoraWs {
  uint16_t *tp, *up, *fr;
  float *pn, *pa, *pb, *gp;
  size_t bytes;
};

// fwd_only: the forward's slices alone (t, the B^T rows, t's partials and
// the forward GEMM's split partials); u and the dA/dB partials take no bytes
LoraWs lora_layout(char* base, int64_t m, int64_t n, int64_t k, int rp, bool fwd_only = false) {
  Slab s{base};
  LoraWs w{};
  w.tp = s.take<uint16_t>(m * rp);
  w.up = s.take<uint16_t>(fwd_only ? 0 : m * rp);
  w.fr = s.take<uint16_t>((fwd_only ? n : std::max(n, k)) * rp);
  const int64_t nt = fwd_only ? lora_plan_nt(m, k, rp).splits
                              : std::max((int64_t)lora_plan_nt(m, k, rp).splits, (int64_t)lora_plan_nt(m, n, rp).splits);
  w.pn = s.take<float>(std::max(nt * round_up(m, 128) * rp, (int64_t)1));
  w.pa = s.take<float>(fwd_only ? 0 : (int64_t)lora_plan_tn(m, k, rp).splits * k * rp);
  w.pb = s.take<float>(fwd_only ? 0 : (int64_t)lora_plan_tn(m, n, rp).splits * n * rp);
  w.gp = s.take<float>(std::max(fwd_only ? gemm_split_floats(m, n, k) : gemm_part_floats(m, n, k), (int64_t)1));
  w.bytes = s.off;
  return w;
}

// Shape limit of the LoRA kernels: 32-bit buffer offsets over one slice.
int check_lora_shapes(lrq_ctx* c, int64_t m, int64_t n, int64_t k, int rp) {
  // the widest slices are those of the two jobs launched together
  const LoraPlan pa = lora_plan_tn(m, k, rp, n), pb = lora_plan_tn(m, n, rp, k);
  const int64_t span = std::max(std::max(16 * std::max(n, k), (pa.per + 256) * k), (pb.per + 256) * n) * 2;
  if (span >= (int64_t)1 << 31)
    return fail(c, LRQ_EUNSUPPORTED, "LoRA shape m=%lld n=%lld k=%lld exceeds 2 GiB per slice",
                (long long)m, (long long)n, (long long)k);
  // t and u keep one arrival counter per 16 tokens in the counter area
  if (m > LRQ_MAX_LORA_TOKENS)
    return fail(c, LRQ_EUNSUPPORTED,
                "LoRA call with m=%lld tokens: the t and u kernels take at most %lld tokens per call (split the "
                "batch)",
                (long long)m, (long long)LRQ_MAX_LORA_TOKENS);
  return LRQ_OK;
}

int check_weight(lrq_ctx* c, const lrq_weight* w, bool gemm) {
  if (!w) return fail(c, LRQ_EINVAL, "weight descriptor is NULL");
  if (w->format != LRQ_FMT_INT4 && w->format != LRQ_FMT_FP8 && w->format != LRQ_FMT_INT8)
    return fail(c, LRQ_EINVAL, "weight format %d is not LRQ_FMT_INT4, LRQ_FMT_FP8 or LRQ_FMT_INT8", w->format);
  if (w->n < 0 || w->k < 0) return fail(c, LRQ_EINVAL, "negative weight shape [%lld, %lld]",
                                        (long long)w->n, (long long)w->k);
  if (w->k % 32 != 0)
    return fail(c, LRQ_EINVAL, "linear weight [%lld, %lld]: the input dim must be a multiple of 32",
                (long long)w->n, (long long)w->k);
  if (w->format != LRQ_FMT_FP8) {
    if (w->group < 32 || (w->group & (w->group - 1)) != 0 || w->k % w->group != 0)
      return fail(c, LRQ_EINVAL,
                  "linear weight [%lld, %lld]: the input dim must be a multiple of the quant block "
                  "(%d), and the block a power of two >= 32",
                  (long long)w->n, (long long)w->k, w->group);
  }
  if (w->layout != LRQ_LAYOUT_ROWS && w->layout != LRQ_LAYOUT_BLOCKED)
    return fail(c, LRQ_EINVAL, "weight layout %d is neither LRQ_LAYOUT_ROWS nor LRQ_LAYOUT_BLOCKED", w->layout);
  if (gemm && w->layout != LRQ_LAYOUT_BLOCKED)
    return fail(c, LRQ_EINVAL, "the fused kernels read LRQ_LAYOUT_BLOCKED weights: call lrq_weight_block once");
  if (gemm && w->n % 8 != 0)
    return fail(c, LRQ_EINVAL, "d_out %lld must be a multiple of 8 for the fused kernels", (long long)w->n);
  if (w->n * w->k > 0 && (!w->data || !w->scales))
    return fail(c, LRQ_EINVAL, "weight data/scales pointer is NULL");
  if (!aligned16(w->data)) return fail(c, LRQ_EINVAL, "weight data must be 16-byte aligned");
  if (w->bias && !aligned16(w->bias)) return fail(c, LRQ_EINVAL, "bias must be 16-byte aligned");
  return LRQ_OK;
}

int begin(lrq_ctx* c) {
  if (!c) return LRQ_EINVAL;
  c->err[0] = 0;
  hipError_t e = hipSetDevice(c->device);
  if (e != hipSuccess) return hip_fail(c, e, "hipSetDevice");
  return LRQ_OK;
}

// Note whether the context's stream is being captured (the hot calls ask
// once per call): a captured graph keeps the workspace's address.
int note_capture(lrq_ctx* c) {
  if (c->captured) return LRQ_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const hipError_t e = hipStreamIsCapturing(c->stream, &cap);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone) c->captured = true;
  return LRQ_OK;
}

#define LRQ_TRY(x)            \
  do {                        \
    int _rc = (x);            \
    if (_rc != LRQ_OK) return _rc; \
  } while (0)

}  // namespace

extern "C" {

int lrq_version(void) { return LRQ_ABI_VERSION; }

int lrq_create(int device, lrq_ctx** out) {
  if (!out) return LRQ_EINVAL;
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || device < 0 || device >= count) return LRQ_EINVAL;
  lrq_ctx* c = new (std::nothrow) lrq_ctx();
  if (!c) return LRQ_ENOMEM;
  c->device = device;
  if (hipSetDevice(device) != hipSuccess) {
    delete c;
    return LRQ_EHIP;
  }
  c->stream = nullptr;  // the null stream until lrq_set_stream says otherwise
  const int rc = init_scratch(device);
  if (rc != LRQ_OK) {
    delete c;
    return rc;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) set_num_cus(prop.multiProcessorCount);
  *out = c;
  return LRQ_OK;
}

int lrq_destroy(lrq_ctx* c) {
  if (!c) return LRQ_OK;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (auto& r : c->pending) {
    (void)hipEventDestroy(r.a);
    (void)hipEventDestroy(r.b);
  }
  for (auto e : c->pool) (void)hipEventDestroy(e);
  if (c->ws_alloc) (void)hipFree(c->ws_alloc);
  for (char* p : c->retired) (void)hipFree(p);
  delete c;
  return LRQ_OK;
}

int lrq_set_stream(lrq_ctx* c, void* stream) {
  LRQ_TRY(begin(c));
  c->stream = reinterpret_cast<hipStream_t>(stream);  // NULL: the device's null stream
  return LRQ_OK;
}

// Reset a counter area after a reported failure, with no kernel running on
// the device: every counter and the flag to zero, the epoch moved past every
// stamp already published (a late t slice of the failed launch may have
// stamped its publication with the epoch of that time), so no stale entry
// matches the next launch's stamp.
static int reset_counters(lrq_ctx* c, uint32_t* cnt) {
  uint32_t ep = 0;
  hipError_t e = hipMemcpy(&ep, cnt + SK_EPOCH, sizeof(ep), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(c, e, "hipMemcpy");
  e = hipMemset(cnt, 0, LRQ_CNT_BYTES);
  if (e != hipSuccess) return hip_fail(c, e, "hipMemset");
  ep += 2;
  e = hipMemcpy(cnt + SK_EPOCH, &ep, sizeof(ep), hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(c, e, "hipMemcpy");
  return LRQ_OK;
}

int lrq_sync(lrq_ctx* c) {
  LRQ_TRY(begin(c));
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) return hip_fail(c, e, "hipStreamSynchronize");
  // a few-token epilogue that gave up waiting for t leaves a flag in the
  // counters (the context's own and the device's scratch array)
  char* scratch = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    scratch = g_scratch[c->device];
  }
  uint32_t* counters[2] = {c->cnt, reinterpret_cast<uint32_t*>(scratch)};
  bool failed = false;
  for (uint32_t* cnt : counters) {
    if (!cnt) continue;
    uint32_t flag = 0;
    e = hipMemcpy(&flag, cnt + SK_FAIL, sizeof(flag), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(c, e, "hipMemcpy");
    failed = failed || flag != 0;
  }
  if (!failed) return LRQ_OK;
  // the late workgroups of the failed launch, and any other stream's use of
  // the scratch array, end before the counters are rewritten
  e = hipDeviceSynchronize();
  if (e != hipSuccess) return hip_fail(c, e, "hipDeviceSynchronize");
  for (uint32_t* cnt : counters)
    if (cnt) LRQ_TRY(reset_counters(c, cnt));
  return fail(c, LRQ_EHIP,
              "a few-token kernel gave up waiting for its t (u) slices: the outputs it wrote are NaN; the flag "
              "is cleared and the counters reset");
}

int lrq_probe_stream_read(lrq_ctx* c, const void* data, int64_t bytes) {
  LRQ_TRY(begin(c));
  if (bytes < 0 || bytes % 16 != 0 || (bytes > 0 && !data) || !aligned16(data))
    return fail(c, LRQ_EINVAL, "the probe reads a 16-byte aligned buffer of a multiple of 16 bytes");
  LRQ_TRY(ensure_ws(c, (size_t)probe_read_grid(bytes) * 4));
  uint32_t* out = reinterpret_cast<uint32_t*>(c->ws);
  const hipError_t e = launch_stream_read(c->stream, data, bytes, out);
  return e == hipSuccess ? LRQ_OK : hip_fail(c, e, "stream_read");
}

int lrq_debug_gemm_path(int path) {
  if (path < 0 || path > 5) return LRQ_EINVAL;
  set_gemm_path(path);
  return LRQ_OK;
}

int lrq_debug_force_wait_timeout(int on) {
  set_force_wait_timeout(on != 0);
  return LRQ_OK;
}

const char* lrq_last_error(const lrq_ctx* c) { return c ? c->err : "null context"; }

// Workspace floats of the mid-size passes at ranks 8 to 32 (multiples of 8)
// that form the
// LoRA factors in their own launch: the factor's slice partials, then the
// tiles' depth-range partials, then (backward) dB's and dA's token-slice
// partials (both jobs counted).
static int64_t fold_fwd_floats(int64_t m, int64_t n, int64_t k, int rp) {
  const int64_t G = (m + 63) / 64, fs = (k + MID_FOLD_KT - 1) / MID_FOLD_KT;
  return round_up(fs * G * 64 * rp, 64) + mid_split_plan(m, n, k).floats;
}
static int64_t fold_bwd_floats(int64_t m, int64_t n, int64_t k, int rp) {
  const int64_t G = (m + 63) / 64, fs = (n + MID_FOLD_KT - 1) / MID_FOLD_KT;
  const LoraPlan tpb = mid_tn_plan(m, n, rp), tpa = mid_tn_plan(m, k, rp);
  return round_up(fs * G * 64 * rp, 64) + round_up(mid_split_plan(m, k, n).floats, 64) +
         (tpb.splits > 1 ? (int64_t)tpb.splits * n * rp : 0) + (tpa.splits > 1 ? (int64_t)tpa.splits * k * rp : 0);
}

int lrq_reserve(lrq_ctx* c, int64_t m, int64_t n, int64_t k, int64_t r) {
  LRQ_TRY(begin(c));
  if (m < 0 || n < 0 || k < 0 || r < 0 || r > 64) return fail(c, LRQ_EINVAL, "bad reserve shape");
  const int rp = (int)round_up(r > 0 ? r : 16, 16);
  size_t need = lora_layout(nullptr, m, n, k, rp).bytes;
  // the fused GEMMs' split partials are not monotonic in the token count
  // (fewer tiles, more depth ranges): their largest size over m' <= m, which
  // peaks at a whole number of 64-token tiles
  const int64_t gp_m = gemm_part_floats(m, n, k);
  int64_t gp_max = gp_m;
  for (int64_t mm = 64; mm < m; mm += 64) gp_max = std::max(gp_max, gemm_part_floats(mm, n, k));
  need += (size_t)(gp_max - gp_m) * 4;
  if (m >= 1) {  // the few-token forward, at up to 16 tokens
    const size_t sk = skinny_ws_bytes(skinny_plan(n, k, rp, get_num_cus()), m < 16 ? m : 16, n, rp);
    if (sk > need) need = sk;
    // the few-token input gradient: its partials (and u's) follow the LoRA workspace
    const int64_t mm = m < 16 ? m : 16;
    const size_t skd = lora_layout(nullptr, mm, n, k, rp).bytes +
                       skinny_ws_bytes(skinny_plan(k, n, rp, get_num_cus()), mm, k, rp);
    if (skd > need) need = skd;
  }
  if (r % 8 == 0 && r > 0 && r <= 32 && m > 16) {
    // the one-launch mid-size passes, at every token count up to m
    const size_t lb = lora_layout(nullptr, m, n, k, rp).bytes;
    for (int64_t mm = 64;; mm += 64) {
      const int64_t mt = mm < m ? mm : m;
      need = std::max(need, (size_t)fold_fwd_floats(mt, n, k, rp) * 4);
      need = std::max(need, lb + (size_t)fold_bwd_floats(mt, n, k, rp) * 4);
      if (mt == m) break;
    }
  }
  const size_t fp8_need = (size_t)round_up(n * 4, 256);
  if (fp8_need > need) need = fp8_need;
  return ensure_ws(c, need);
}

int lrq_quantize_int4(lrq_ctx* c, const float* w, int64_t n, int64_t k, int64_t group,
                      uint8_t* packed, float* scales) {
  LRQ_TRY(begin(c));
  if (n < 0 || k < 0) return fail(c, LRQ_EINVAL, "negative shape");
  if (group < 32 || group > 2048 || (group & (group - 1)) != 0)
    return fail(c, LRQ_EINVAL, "quant block %lld must be a power of two in [32, 2048]", (long long)group);
  if (k % group != 0)
    return fail(c, LRQ_EINVAL,
                "linear weight [%lld, %lld]: the input dim must be a multiple of the quant block (%lld)",
                (long long)n, (long long)k, (long long)group);
  if (!aligned16(w) || !aligned16(packed)) return fail(c, LRQ_EINVAL, "w and packed must be 16-byte aligned");
  return run(c, KID_QUANT_INT4, "quantize_int4",
             [&] { return launch_quantize_int4(c->stream, w, n, k, (int)group, packed, scales); });
}

int lrq_quantize_int8(lrq_ctx* c, const float* w, int64_t n, int64_t k, int64_t group, int8_t* q,
                      float* scales) {
  LRQ_TRY(begin(c));
  if (n < 0 || k < 0) return fail(c, LRQ_EINVAL, "negative shape");
  if (group < 32 || group > 2048 || (group & (group - 1)) != 0)
    return fail(c, LRQ_EINVAL, "quant block %lld must be a power of two in [32, 2048]", (long long)group);
  if (k % group != 0)
    return fail(c, LRQ_EINVAL,
                "linear weight [%lld, %lld]: the input dim must be a multiple of the quant block (%lld)",
                (long long)n, (long long)k, (long long)group);
  if (n * k > 0 && (!w || !q || !scales)) return fail(c, LRQ_EINVAL, "int8 quantize: NULL pointer");
  if (!aligned16(w) || !aligned16(q)) return fail(c, LRQ_EINVAL, "w and q must be 16-byte aligned");
  return run(c, KID_QUANT_INT8, "quantize_int8",
             [&] { return launch_quantize_int8(c->stream, w, n, k, (int)group, q, scales); });
}

int lrq_requantize_fp8_int4(lrq_ctx* c, const uint8_t* bytes, const float* scale, int per_channel, int64_t n,
                            int64_t k, int64_t group, uint8_t* packed, float* scales) {
  LRQ_TRY(begin(c));
  if (n < 0 || k < 0) return fail(c, LRQ_EINVAL, "negative shape");
  if (group < 32 || group > 2048 || (group & (group - 1)) != 0)
    return fail(c, LRQ_EINVAL, "quant block %lld must be a power of two in [32, 2048]", (long long)group);
  if (k % group != 0)
    return fail(c, LRQ_EINVAL,
                "linear weight [%lld, %lld]: the input dim must be a multiple of the quant block (%lld)",
                (long long)n, (long long)k, (long long)group);
  if (n * k > 0 && (!bytes || !scale || !packed || !scales))
    return fail(c, LRQ_EINVAL, "fp8 requantize: NULL pointer");
  if (!aligned16(bytes) || !aligned16(packed)) return fail(c, LRQ_EINVAL, "bytes and packed must be 16-byte aligned");
  return run(c, KID_QUANT_INT4, "quantize_int4", [&] {
    return launch_requantize_fp8_int4(c->stream, bytes, scale, per_channel ? 1 : 0, n, k, (int)group, packed,
                                      scales);
  });
}

int lrq_quantize_fp8(lrq_ctx* c, const float* w, int64_t n, int64_t k, int per_channel,
                     uint8_t* bytes, float* scales) {
  LRQ_TRY(begin(c));
  if (n < 0 || k < 0 || k % 4 != 0) return fail(c, LRQ_EINVAL, "fp8 quantize needs k %% 4 == 0");
  if (!aligned16(w) || !aligned16(bytes)) return fail(c, LRQ_EINVAL, "w and bytes must be 16-byte aligned");
  LRQ_TRY(ensure_ws(c, (size_t)round_up((n > 0 ? n : 1) * 4, 256)));
  float* amax = reinterpret_cast<float*>(c->ws);
  return run(c, KID_QUANT_FP8, "quantize_fp8", [&] {
    return launch_quantize_fp8(c->stream, w, n, k, per_channel, bytes, scales, amax);
  });
}

int lrq_weight_blocked_size(int format, int64_t n, int64_t k, int64_t group, int64_t* data_bytes,
                            int64_t* scale_count) {
  if ((format != LRQ_FMT_INT4 && format != LRQ_FMT_FP8 && format != LRQ_FMT_INT8) || n < 0 || k < 0 ||
      !data_bytes || !scale_count)
    return LRQ_EINVAL;
  const bool gs = format != LRQ_FMT_FP8;  // group scales
  if (gs && (group < 32 || (group & (group - 1)) != 0 || k % group != 0)) return LRQ_EINVAL;
  blocked_sizes(format, n, k, gs ? group : 64, data_bytes, scale_count);
  return LRQ_OK;
}

int lrq_weight_block(lrq_ctx* c, const lrq_weight* w, uint8_t* data_out, float* scales_out) {
  LRQ_TRY(begin(c));
  LRQ_TRY(check_weight(c, w, false));
  if (w->layout != LRQ_LAYOUT_ROWS) return fail(c, LRQ_EINVAL, "lrq_weight_block takes a LRQ_LAYOUT_ROWS weight");
  if (w->format != LRQ_FMT_FP8 && ((w->group & (w->group - 1)) != 0))
    return fail(c, LRQ_EINVAL, "quant block %d must be a power of two", w->group);
  if (!aligned16(data_out)) return fail(c, LRQ_EINVAL, "data_out must be 16-byte aligned");
  if (w->format != LRQ_FMT_FP8 && !scales_out) return fail(c, LRQ_EINVAL, "scales_out is NULL");
  return run(c, KID_BLOCK, "weight_block", [&] { return launch_block(c->stream, w, data_out, scales_out); });
}

int lrq_dequant(lrq_ctx* c, const lrq_weight* w, float* out) {
  LRQ_TRY(begin(c));
  LRQ_TRY(check_weight(c, w, false));
  if (!aligned16(out)) return fail(c, LRQ_EINVAL, "out must be 16-byte aligned");
  return run(c, KID_DEQUANT, "dequant", [&] { return launch_dequant(c->stream, w, out, false); });
}

int lrq_dequant_bf16(lrq_ctx* c, const lrq_weight* w, uint16_t* out) {
  LRQ_TRY(begin(c));
  LRQ_TRY(check_weight(c, w, false));
  if (!aligned16(out)) return fail(c, LRQ_EINVAL, "out must be 16-byte aligned");
  return run(c, KID_DEQUANT, "dequant_bf16", [&] { return launch_dequant(c->stream, w, out, true); });
}

static GemmArgs gemm_args(const lrq_weight* w, bool bwd, const uint16_t* act, int64_t m, uint16_t* out) {
  GemmArgs g{};
  g.act = act;
  g.m = m;
  g.l = bwd ? w->n : w->k;
  g.e = bwd ? w->k : w->n;
  g.wk = w->k;
  // forward: the row section of the blocked layout; backward: the transposed
  // section (and, int4 and int8, its scale table) that follows it
  int64_t db = 0, sc = 0;
  if (bwd) blocked_sections(w->format, w->n, w->k, w->group, &db, &sc);
  g.wdata = reinterpret_cast<const uint8_t*>(w->data) + db;
  g.wscale = w->scales + sc;
  g.group = w->group;
  g.gshift = 0;
  while (w->group > 0 && (1 << g.gshift) < w->group) ++g.gshift;
  g.per_channel = w->per_channel;
  g.nib = 0x0f0f0f0fu;
  g.bias = bwd ? nullptr : w->bias;
  g.out = out;
  g.tn_da = -1;
  return g;
}

static int check_gemm(lrq_ctx* c, const lrq_weight* w, int64_t m) {
  LRQ_TRY(check_weight(c, w, true));
  if (m < 0) return fail(c, LRQ_EINVAL, "negative token count");
  int64_t wbytes = 0, nscales = 0;
  blocked_sections(w->format, w->n, w->k, w->group, &wbytes, &nscales);
  if (wbytes >= (int64_t)1 << 31)
    return fail(c, LRQ_EUNSUPPORTED, "packed weight of %lld bytes: the fused kernels address at most 2 GiB",
                (long long)wbytes);
  if (w->n <= 0 || w->k <= 0)
    return fail(c, LRQ_EINVAL, "the fused kernels need d_out > 0 and d_in > 0 (got [%lld, %lld])",
                (long long)w->n, (long long)w->k);
  return LRQ_OK;
}

// Where the forward's workspace comes from: the context's (grown on demand)
// or, for lrq_lora_fwd_noalloc, the device's static scratch array.
// Both start with the few-token kernels' arrival counters (LRQ_CNT_BYTES).
struct WsSource {
  bool scratch;
  char* base;
};

static int acquire_ws(lrq_ctx* c, WsSource* src, size_t bytes, char** out, uint32_t** cnt) {
  if (!src->scratch) {
    LRQ_TRY(ensure_ws(c, bytes));
    *out = c->ws;
    *cnt = c->cnt;
    return LRQ_OK;
  }
  const size_t cap = (size_t)LRQ_NOALLOC_SCRATCH_BYTES - LRQ_CNT_BYTES;
  if (bytes > cap)
    return fail(c, LRQ_EINVAL,
                "lrq_lora_fwd_noalloc: this shape needs %zu bytes of scratch, more than its fixed %zu; use "
                "lrq_lora_fwd",
                bytes, cap);
  *cnt = reinterpret_cast<uint32_t*>(src->base);
  *out = src->base + LRQ_CNT_BYTES;
  return LRQ_OK;
}

static int fwd_impl(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, int64_t m, const uint16_t* a,
                    const uint16_t* b, int64_t r, float scaling, uint16_t* y, uint16_t* t_out, WsSource* src) {
  LRQ_TRY(begin(c));
  LRQ_TRY(note_capture(c));
  LRQ_TRY(check_gemm(c, w, m));
  if (!aligned16(x) || !aligned16(y)) return fail(c, LRQ_EINVAL, "x and y must be 16-byte aligned");
  forget_pass(c, false);
  const int fmt = w->format;
  const int64_t wk = w->k;
  const bool lora = a != nullptr && b != nullptr && r > 0;
  GemmArgs ga = gemm_args(w, false, x, m, y);
  if (lora) {
    if (r > 64) return fail(c, LRQ_EINVAL, "rank %lld outside [1, 64]", (long long)r);
    if (!aligned16(b)) return fail(c, LRQ_EINVAL, "B must be 16-byte aligned");
  }
  char* ws = nullptr;
  uint32_t* cnt = nullptr;
  if (m >= 1 && m <= 16) {
    // few tokens: one launch streams the packed weight once (split-k
    // partials, t's partials alongside); the last arrival at each block row
    // finishes it
    const int rp = lora ? (int)round_up(r, 16) : 0;
    const SkinnyPlan p = skinny_plan(w->n, w->k, rp, get_num_cus());
    LRQ_TRY(acquire_ws(c, src, skinny_ws_bytes(p, m, w->n, rp), &ws, &cnt));
    float* part = reinterpret_cast<float*>(ws);
    float* tpart = part + round_up((int64_t)p.S * m * w->n, 64);
    if (lora) {
      ga.lw = b;
      ga.r = (int)r;
      ga.rp = rp;
    }
    const uint16_t* ta = lora ? a : nullptr;
    uint16_t* tt = lora ? t_out : nullptr;
    return run_hot(c, KID_FWD_MAIN, "fwd_main", [=] {
      return launch_skinny(c->stream, fmt, false, ga, ta, p, part, tpart, cnt, scaling, tt);
    });
  }
  if (lora) {
    const int rp = (int)round_up(r, 16);
    LRQ_TRY(check_lora_shapes(c, m, w->n, w->k, rp));
    // mid-size tiles at ranks 8 to 32 (multiples of 8): t is formed in the same launch by
    // workgroups ahead of the tiles (no side launch)
    const int64_t G = (m + 63) / 64, fs = (w->k + MID_FOLD_KT - 1) / MID_FOLD_KT;
    // (and the tiles' depth ranges, if any: partials after t's, counters
    // after the fold's)
    const MidSplit ms = mid_split_plan(m, w->n, w->k);
    if (r % 8 == 0 && r <= 32 && gemm_mid_tokens(m, w->n, w->k) > 0 && aligned16(a) && t_out && aligned16(t_out) &&
        2 * G + ms.tiles <= SK_MAX_NB) {
      const int64_t fp = round_up(fs * G * 64 * rp, 64);
      LRQ_TRY(acquire_ws(c, src, (size_t)(fp + ms.floats) * 4, &ws, &cnt));
      ga.fold = force_wait_timeout() ? -1 : 1;
      ga.fold_slices = (int)fs;
      ga.fold_wgs = (int)round_up(fs * G, 8);
      ga.fpart = reinterpret_cast<float*>(ws);
      ga.fcnt = cnt;
      ga.part = ms.floats > 0 ? ga.fpart + fp : nullptr;
      ga.mcnt = cnt + 2 * G;
      ga.lact = a;
      ga.lw = b;
      ga.fscale = scaling;
      ga.fout = t_out;
      ga.fout_ld = (int)r;
      ga.r = (int)r;
      ga.rp = rp;
      return run_hot(c, KID_FWD_MAIN, "fwd_main", [=] { return launch_fwd(c->stream, fmt, ga); });
    }
    LRQ_TRY(acquire_ws(c, src, lora_layout(nullptr, m, w->n, w->k, rp, true).bytes, &ws, &cnt));
    LoraWs lw = lora_layout(ws, m, w->n, w->k, rp, true);
    // t = s . x . A   (bf16 [m, rp] for the fused step, [m, r] for the caller)
    const LoraPlan pt = lora_plan_nt(m, w->k, rp);
    // fp8: B^T divided by the weight scale (the GEMM scales base + LoRA)
    const bool f8 = w->format == LRQ_FMT_FP8;
    const NtFinish fin{cnt,  scaling, (int)r, lw.tp,  t_out, b, w->n, 0,
                       lw.fr, f8 ? w->scales : nullptr, (f8 && w->per_channel) ? 1 : 0};
    float* pn = lw.pn;
    LRQ_TRY(run_hot(c, KID_LORA_T, "lora_t", [=] {
      return launch_lora_nt(c->stream, x, a, false, r, (int)r, m, wk, rp, pt, pn, fin);
    }));
    ga.lact = lw.tp;
    ga.lw = lw.fr;
    ga.r = (int)r;
    ga.rp = rp;
    ga.part = lw.gp;
    ga.mcnt = cnt;
  } else {
    const int64_t pf = gemm_split_floats(m, w->n, w->k);
    if (pf > 0) {
      LRQ_TRY(acquire_ws(c, src, (size_t)pf * 4, &ws, &cnt));
      ga.part = reinterpret_cast<float*>(ws);
      ga.mcnt = cnt;
    }
  }
  return run_hot(c, KID_FWD_MAIN, "fwd_main", [=] { return launch_fwd(c->stream, fmt, ga); });
}

int lrq_quant_matmul_t(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, int64_t m, uint16_t* y) {
  WsSource src{false, nullptr};
  return fwd_impl(c, w, x, m, nullptr, nullptr, 0, 1.0f, y, nullptr, &src);
}

int lrq_lora_fwd(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, int64_t m, const uint16_t* a,
                 const uint16_t* b, int64_t r, float scaling, uint16_t* y, uint16_t* t_out) {
  if (c && (r < 1 || r > 64 || !a || !b)) {
    c->err[0] = 0;
    return fail(c, LRQ_EINVAL, "lrq_lora_fwd needs A, B and 1 <= r <= 64 (got r=%lld)", (long long)r);
  }
  WsSource src{false, nullptr};
  return fwd_impl(c, w, x, m, a, b, r, scaling, y, t_out, &src);
}

int lrq_lora_fwd_noalloc(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, int64_t m, const uint16_t* a,
                         const uint16_t* b, int64_t r, float scaling, uint16_t* y, uint16_t* t_out) {
  if (!c) return LRQ_EINVAL;
  c->err[0] = 0;
  if (r < 1 || r > 64 || !a || !b)
    return fail(c, LRQ_EINVAL, "lrq_lora_fwd_noalloc needs A, B and 1 <= r <= 64 (got r=%lld)", (long long)r);
  char* base = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    base = (c->device >= 0 && c->device < kMaxDevices) ? g_scratch[c->device] : nullptr;
  }
  if (!base) return fail(c, LRQ_EHIP, "no scratch address for device %d", c->device);
  WsSource src{true, base};
  // no per-kernel event brackets: creating their events could allocate
  const bool prof = c->prof;
  c->prof = false;
  const int rc = fwd_impl(c, w, x, m, a, b, r, scaling, y, t_out, &src);
  c->prof = prof;
  return rc;
}

// The input gradient: the few-token path for m <= 16 (partials at `skpart`),
// else the fused GEMM.
static hipError_t launch_dx(lrq_ctx* c, int fmt, int64_t wn, int64_t wk, const GemmArgs& ga, int64_t m,
                            float* skpart) {
  if (m >= 1 && m <= 16) {
    const SkinnyPlan p = skinny_plan(wk, wn, 0, get_num_cus());
    return launch_skinny(c->stream, fmt, true, ga, nullptr, p, skpart, nullptr, c->cnt, 1.0f, nullptr);
  }
  return launch_bwd(c->stream, fmt, ga);
}

// workspace bytes of the few-token input gradient's partials (0 for m > 16)
static size_t skinny_dx_bytes(const lrq_weight* w, int64_t m) {
  if (m < 1 || m > 16) return 0;
  return skinny_ws_bytes(skinny_plan(w->k, w->n, 0, get_num_cus()), m, w->k, 0);
}

static int bwd_impl(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, const uint16_t* dy, int64_t m,
                    const uint16_t* a, const uint16_t* b, int64_t r, float scaling, const uint16_t* t,
                    uint16_t* dx, float* da, float* db) {
  LRQ_TRY(begin(c));
  LRQ_TRY(note_capture(c));
  LRQ_TRY(check_gemm(c, w, m));
  if (!aligned16(dy)) return fail(c, LRQ_EINVAL, "dy must be 16-byte aligned");
  forget_pass(c, true);
  const int fmt = w->format;
  const int64_t wn = w->n, wk = w->k;
  if (dx && !aligned16(dx)) return fail(c, LRQ_EINVAL, "dx must be 16-byte aligned");
  const bool lora = a != nullptr && b != nullptr && r > 0;
  GemmArgs ga = gemm_args(w, true, dy, m, dx);
  if (lora) {
    if (r > 64) return fail(c, LRQ_EINVAL, "rank %lld outside [1, 64]", (long long)r);
    if ((da && (!x || !aligned16(x))) || (db && !t))
      return fail(c, LRQ_EINVAL, "dA needs x and dB needs t (16-byte aligned)");
    if (!aligned16(b)) return fail(c, LRQ_EINVAL, "B must be 16-byte aligned");
    const int rp = (int)round_up(r, 16);
    LRQ_TRY(check_lora_shapes(c, m, w->n, w->k, rp));
    const bool few = dx && m >= 1 && m <= 16;
    const SkinnyPlan sp = skinny_plan(w->k, w->n, rp, get_num_cus());
    const size_t lbytes = lora_layout(nullptr, m, w->n, w->k, rp).bytes;
    // mid-size tiles at ranks 8 to 32 (multiples of 8): u is formed in the input gradient's
    // launch by workgroups ahead of the tiles (partials after the LoRA
    // workspace)
    const int64_t G = (m + 63) / 64, fs = (w->n + MID_FOLD_KT - 1) / MID_FOLD_KT;
    const bool fold = !few && dx && r % 8 == 0 && r <= 32 && gemm_mid_tokens(m, w->k, w->n) > 0 && aligned16(a) &&
                      2 * G + mid_split_plan(m, w->k, w->n).tiles <= SK_MAX_NB;
    // and the weight gradients by workgroups after its tiles, in token
    // slices that fit its LDS (their counters after the fold's, partials
    // after u's)
    const LoraPlan tpb = fold ? mid_tn_plan(m, w->n, rp) : LoraPlan{}, tpa = fold ? mid_tn_plan(m, w->k, rp) : LoraPlan{};
    const int64_t tb_floats = (db && tpb.splits > 1) ? (int64_t)tpb.splits * w->n * rp : 0;
    const int64_t ta_floats = (da && tpa.splits > 1) ? (int64_t)tpa.splits * w->k * rp : 0;
    // the tiles' depth ranges, if any (their partials and counters first)
    const MidSplit ms = fold ? mid_split_plan(m, w->k, w->n) : MidSplit{1, 0, 0, 0};
    const bool fold_tn = fold && (da || db) && tpb.splits > 0 && tpa.splits > 0 &&
                         2 * G + ms.tiles + TN_WAVES * ((db ? tpb.tiles : 0) + (da ? tpa.tiles : 0)) <= SK_MAX_NB;
    const int64_t fp_floats = round_up(fs * G * 64 * rp, 64);
    const int64_t ms_floats = round_up(ms.floats, 64);
    const size_t fbytes = fold ? (size_t)(fp_floats + ms_floats + (fold_tn ? tb_floats + ta_floats : 0)) * 4 : 0;
    LRQ_TRY(ensure_ws(c, lbytes + (few ? skinny_ws_bytes(sp, m, w->k, rp) : fbytes)));
    LoraWs ws = lora_layout(c->ws, m, w->n, w->k, rp);
    ga.r = (int)r;
    ga.rp = rp;
    if (few) {
      // few tokens: u = s . dy . B^T (bf16 [m, rp], dA's factor) comes out
      // of the input gradient's own launch, as t does in the forward
      float* part = reinterpret_cast<float*>(c->ws + lbytes);
      float* tpart = part + round_up((int64_t)sp.S * m * w->k, 64);
      ga.lw = a;
      uint16_t* up = ws.up;
      // and dA = x^T . u, dB = t^T . dy in the same launch: dB by the split
      // workgroups (nothing to wait for), dA by each block row's epilogue
      // once u is in
      const SkGrads gr{da ? x : nullptr, db ? t : nullptr, da, db};
      LRQ_TRY(run_hot(c, KID_BWD_DX, "bwd_dx", [=] {
        return launch_skinny(c->stream, fmt, true, ga, b, sp, part, tpart, c->cnt, scaling, up, gr);
      }));
      return LRQ_OK;
    } else if (fold) {
      // u (stored to the workspace for dA) from the fold's workgroups
      ga.fold = force_wait_timeout() ? -1 : 1;
      ga.fold_slices = (int)fs;
      ga.fold_wgs = (int)round_up(fs * G, 8);
      ga.fpart = reinterpret_cast<float*>(c->ws + lbytes);
      ga.fcnt = c->cnt;
      ga.lact = b;
      ga.lw = a;
      ga.fscale = scaling;
      ga.fout = ws.up;
      ga.fout_ld = rp;
      ga.part = ms.floats > 0 ? ga.fpart + fp_floats : nullptr;
      ga.mcnt = c->cnt + 2 * G;
      if (fold_tn) {
        // dB = t^T . dy first (nothing to wait for), then dA = x^T . u
        float* tpart = ga.fpart + fp_floats + ms_floats;
        uint32_t* tcnt = c->cnt + 2 * G + ms.tiles;
        int nj = 0;
        if (db) {
          ga.tj[nj++] = tn_args(TnSpec{dy, t, r, m, w->n, (int)r, tpb, tpart, db, 1, w->n}, tcnt);
          tpart += tb_floats;
          tcnt += TN_WAVES * tpb.tiles;
        }
        if (da) {
          ga.tn_da = nj;
          ga.tj[nj++] = tn_args(TnSpec{x, ws.up, rp, m, w->k, (int)r, tpa, tpart, da, r, 1}, tcnt);
        }
        ga.tn_blocks = ga.tj[0].blocks + ga.tj[1].blocks;
      }
      LRQ_TRY(run_hot(c, KID_BWD_DX, "bwd_dx", [=] { return launch_bwd(c->stream, fmt, ga); }));
      if (fold_tn) return LRQ_OK;
    } else {
      // u = s . dy . B^T   (bf16 [m, rp]: the dx epilogue operand and dA's factor)
      const LoraPlan pu = lora_plan_nt(m, w->n, rp);
      const LoraWs wsv = ws;
      LRQ_TRY(run_hot(c, KID_LORA_U, "lora_u", [=] {
        // and A [k, r] padded to [k, rp]: the dx GEMM's weight-side LoRA rows
        const NtFinish fin{c->cnt, scaling, (int)r, wsv.up, nullptr, a, wk, 1, wsv.fr, nullptr, 0};
        return launch_lora_nt(c->stream, dy, b, true, wn, (int)r, m, wn, rp, pu, wsv.pn, fin);
      }));
      ga.lact = ws.up;
      ga.lw = ws.fr;
      ga.part = ws.gp;
      ga.mcnt = c->cnt;
      if (dx) LRQ_TRY(run_hot(c, KID_BWD_DX, "bwd_dx", [=] { return launch_bwd(c->stream, fmt, ga); }));
    }
    // dA = x^T . u -> f32 [k, r] and dB = t^T . dy -> f32 [r, n]: token-slice
    // partials of both in one launch (dB's longer workgroups dispatched
    // first), each column tile finished by its last slice
    TnSpec specs[2] = {};
    int nj = 0;
    // (planned together when both run: fewer, longer slices than either
    // alone, so the partials reserved for the single-job plans suffice)
    const int64_t ob = da ? w->k : 0, oa = db ? w->n : 0;
    if (db) specs[nj++] = TnSpec{dy, t, r, m, w->n, (int)r, lora_plan_tn(m, w->n, rp, ob), ws.pb, db, 1, w->n};
    if (da) specs[nj++] = TnSpec{x, ws.up, rp, m, w->k, (int)r, lora_plan_tn(m, w->k, rp, oa), ws.pa, da, r, 1};
    if (nj) {
      const int kid = nj == 2 ? KID_LORA_DADB : (db ? KID_LORA_DB : KID_LORA_DA);
      const TnSpec s0 = specs[0], s1 = specs[1];
      LRQ_TRY(run_hot(c, kid, kNames[kid], [=] {
        const TnSpec sp[2] = {s0, s1};
        return launch_lora_tn(c->stream, sp, nj, rp, c->cnt);
      }));
    }
    return LRQ_OK;
  }
  if (!dx) return LRQ_OK;
  const int64_t pf = (m >= 1 && m <= 16) ? 0 : gemm_split_floats(m, w->k, w->n);
  LRQ_TRY(ensure_ws(c, std::max((size_t)pf * 4, skinny_dx_bytes(w, m))));
  if (pf > 0) {
    ga.part = reinterpret_cast<float*>(c->ws);
    ga.mcnt = c->cnt;
  }
  float* skpart = reinterpret_cast<float*>(c->ws);
  return run_hot(c, KID_BWD_DX, "bwd_dx", [=] { return launch_dx(c, fmt, wn, wk, ga, m, skpart); });
}

int lrq_quant_matmul_t_bwd(lrq_ctx* c, const lrq_weight* w, const uint16_t* dy, int64_t m, uint16_t* dx) {
  return bwd_impl(c, w, nullptr, dy, m, nullptr, nullptr, 0, 1.0f, nullptr, dx, nullptr, nullptr);
}

int lrq_lora_bwd(lrq_ctx* c, const lrq_weight* w, const uint16_t* x, const uint16_t* dy, int64_t m,
                 const uint16_t* a, const uint16_t* b, int64_t r, float scaling, const uint16_t* t,
                 uint16_t* dx, float* da, float* db) {
  if (c && (r < 1 || r > 64 || !a || !b)) {
    c->err[0] = 0;
    return fail(c, LRQ_EINVAL, "lrq_lora_bwd needs A, B and 1 <= r <= 64 (got r=%lld)", (long long)r);
  }
  return bwd_impl(c, w, x, dy, m, a, b, r, scaling, t, dx, da, db);
}

int lrq_profile_enable(lrq_ctx* c, int on) {
  LRQ_TRY(begin(c));
  c->prof = on != 0;
  return LRQ_OK;
}

int lrq_profile_reset(lrq_ctx* c) {
  LRQ_TRY(begin(c));
  LRQ_TRY(flush_profile(c));
  for (int i = 0; i < KID_COUNT; ++i) {
    c->total_ms[i] = 0.0;
    c->launches[i] = 0;
  }
  return LRQ_OK;
}

int lrq_profile_count(void) { return KID_COUNT; }

int lrq_profile_relaunch(lrq_ctx* c, int kid, int n) {
  LRQ_TRY(begin(c));
  if (kid < 0 || kid >= KID_COUNT || n < 0) return fail(c, LRQ_EINVAL, "kernel id %d or count %d out of range", kid, n);
  if (!c->last[kid]) return fail(c, LRQ_EINVAL, "no launch of kernel %s on this context to repeat", kNames[kid]);
  for (int i = 0; i < n; ++i) {
    const hipError_t e = c->last[kid]();
    if (e != hipSuccess) return hip_fail(c, e, kNames[kid]);
  }
  return LRQ_OK;
}

const char* lrq_profile_name(int kid) { return (kid >= 0 && kid < KID_COUNT) ? kNames[kid] : ""; }

int lrq_profile_read(lrq_ctx* c, int kid, double* total_ms, int64_t* launches) {
  LRQ_TRY(begin(c));
  if (kid < 0 || kid >= KID_COUNT) return fail(c, LRQ_EINVAL, "kernel id %d out of range", kid);
  LRQ_TRY(flush_profile(c));
  if (total_ms) *total_ms = c->total_ms[kid];
  if (launches) *launches = c->launches[kid];
  return LRQ_OK;
}

}  // extern "C"
