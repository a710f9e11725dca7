// C ABI of the gfx950 Q4_0 / FP16 matmul library (declared in
// include/hypno_hip.h).  Validates arguments, picks a kernel by shape and
// alignment, and owns the device-side state: per-device streams and staging
// buffers for the host-slice entry points, per-stream GEMM workspaces, and the
// weight-residency registry.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "../../include/hypno_hip.h"
#include "common.hpp"

namespace {

using namespace hypno;

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return status;
}

int hip_fail(hipError_t e, const char* what) {
  const int st = e == hipErrorOutOfMemory ? HYPNO_HIP_ENOMEM : HYPNO_HIP_EDEVICE;
  return fail(st, "%s: %s", what, hipGetErrorString(e));
}

// Token counts 2 .. kSkinnyMaxBatch go to the weight-streaming MFMA kernel,
// larger ones (from kGemmMinBatch) to the tiled prefill GEMM.
constexpr size_t kSkinnyMaxBatch = 64;
constexpr size_t kGemmMinBatch = 16;

struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
};

// Grow-only device buffer; `sync` is the stream whose queued work may still use
// the old allocation.
hipError_t ensure(DevBuf& b, size_t bytes, hipStream_t sync) {
  if (b.cap >= bytes && b.p) return hipSuccess;
  if (b.p) {
    hipError_t e = hipStreamSynchronize(sync);
    if (e != hipSuccess) return e;
    (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
  }
  const size_t want = bytes < 256 ? 256 : bytes;
  hipError_t e = hipMalloc(&b.p, want);
  if (e != hipSuccess) {
    b.p = nullptr;
    return e;
  }
  b.cap = want;
  return hipSuccess;
}

// Grow-only page-locked host buffer (hipHostMalloc).  Host-slice calls stage
// x, bias and y through it: a copy from page-locked memory is a plain DMA,
// where the runtime stages a pageable one itself with host-side waits.
constexpr size_t kPinnedMax = (size_t)8 << 20;  // larger slices are copied directly
hipError_t ensure_host(DevBuf& b, size_t bytes, hipStream_t sync) {
  if (b.cap >= bytes && b.p) return hipSuccess;
  if (b.p) {
    hipError_t e = hipStreamSynchronize(sync);
    if (e != hipSuccess) return e;
    (void)hipHostFree(b.p);
    b.p = nullptr;
    b.cap = 0;
  }
  const size_t want = (bytes < 65536 ? 65536 : bytes + 4095) / 4096 * 4096;
  hipError_t e = hipHostMalloc(&b.p, want, hipHostMallocMapped);
  if (e != hipSuccess) {
    b.p = nullptr;
    return e;
  }
  b.cap = want;
  return hipSuccess;
}

// Host -> device copy of a host slice on stream s, through the page-locked
// buffer `pin` when it is small enough.
hipError_t upload(void* dst, const void* src, size_t bytes, DevBuf& pin, hipStream_t s) {
  if (bytes > kPinnedMax) return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s);
  hipError_t e = ensure_host(pin, bytes, s);
  if (e != hipSuccess) return e;
  memcpy(pin.p, src, bytes);
  return hipMemcpyAsync(dst, pin.p, bytes, hipMemcpyHostToDevice, s);
}

// Workspace of one (device, stream).  Its mutex is held from the size check
// through the last launch of a call, so two threads calling on one stream
// neither free a buffer the other is about to launch with nor interleave
// their multi-kernel sequences (pre-pass, GEMM, reduction); a buffer is only
// replaced after the stream has drained.
struct StreamWs {
  std::mutex mu;
  DevBuf buf;
};

struct DeviceState {
  bool init = false;
  int cus = 256;
  hipStream_t stream = nullptr;  // used by the host-slice entry points
  DevBuf w, x, y, bias;          // host-slice staging
  DevBuf hx, hy, hbias;          // page-locked host staging of x, y, bias
  std::map<hipStream_t, std::unique_ptr<StreamWs>> workspaces;
};

struct Registered {
  void* dev_ptr;
  size_t len;
  int device;
};

std::mutex g_host_mu;  // serialises host-slice calls (staging buffers, registry copies)
std::mutex g_mu;       // guards the maps below and the per-stream workspaces
std::map<int, DeviceState> g_dev;
std::map<const uint8_t*, Registered> g_weights;

int current_device(int* dev) {
  hipError_t e = hipGetDevice(dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  return HYPNO_HIP_OK;
}

// Caller holds g_mu.
int device_state(DeviceState** out) {
  int dev = 0;
  int st = current_device(&dev);
  if (st) return st;
  DeviceState& d = g_dev[dev];
  if (!d.init) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
      d.cus = cus;
    hipError_t e = hipStreamCreateWithFlags(&d.stream, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreate");
    d.init = true;
  }
  *out = &d;
  return HYPNO_HIP_OK;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// A locked workspace: valid (and exclusively this caller's on its stream)
// until the object goes out of scope.
struct WsLock {
  std::unique_lock<std::mutex> lk;
  void* p = nullptr;
};

// Locks stream s's workspace on the device of `ds` and grows it to `bytes`.
int lock_workspace(DeviceState* ds, hipStream_t s, size_t bytes, WsLock& out,
                   const char* what) {
  StreamWs* w = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    std::unique_ptr<StreamWs>& slot = ds->workspaces[s];
    if (!slot) slot.reset(new StreamWs());
    w = slot.get();
  }
  out.lk = std::unique_lock<std::mutex>(w->mu);
  hipError_t e = ensure(w->buf, bytes, s);
  if (e != hipSuccess) return hip_fail(e, what);
  out.p = w->buf.p;
  return HYPNO_HIP_OK;
}

// [a, a + na) and [b, b + nb) share a byte (empty ranges share none).
bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  if (!a || !b || !na || !nb) return false;
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + nb && y < x + na;
}

// The output of a device call may not share memory with any of its inputs
// (the reference takes `y: &mut [f32]` beside shared borrows of the rest,
// which Rust keeps disjoint).
int check_disjoint(const float* y, size_t ybytes, const void* w, size_t wbytes, const float* x,
                   size_t xbytes, const float* bias, size_t bbytes) {
  if (overlaps(y, ybytes, x, xbytes) || overlaps(y, ybytes, w, wbytes) ||
      overlaps(y, ybytes, bias, bbytes))
    return fail(HYPNO_HIP_EINVAL, "y overlaps an input buffer");
  return HYPNO_HIP_OK;
}

bool mul_overflows(size_t a, size_t b) { return a != 0 && b > SIZE_MAX / a; }

// --- dispatch on device pointers (caller holds no lock) ---------------------

// A fixed device buffer standing in for the per-stream workspace (the
// no-allocation entry point): `ptr` holds `bytes`; `cus` is the device's CU
// count.
struct FixedScratch {
  void* ptr = nullptr;
  size_t bytes = 0;
  int cus = 256;
};

int q4_0_dev(float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
             size_t n, size_t m, size_t batch, hipStream_t s,
             const FixedScratch* fixed = nullptr) {
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  if (!y || !x) return fail(HYPNO_HIP_EINVAL, "y and x must not be NULL");
  if (!w && w_len) return fail(HYPNO_HIP_EINVAL, "w_q is NULL but w_len > 0");
  if (mul_overflows(n, batch) || mul_overflows(m, batch) || mul_overflows(n, m))
    return fail(HYPNO_HIP_EINVAL, "shape overflows size_t");
  int st = check_disjoint(y, n * batch * 4, w, w_len, x, m * batch * 4, bias, bias ? n * 4 : 0);
  if (st) return st;
  int cus = 256;
  DeviceState* ds = nullptr;
  if (fixed) {
    cus = fixed->cus;
  } else {
    std::lock_guard<std::mutex> g(g_mu);
    st = device_state(&ds);
    if (st) return st;
    cus = ds->cus;
  }
  // The call's scratch memory: the stream's workspace (locked for the span
  // of the launches), or the fixed buffer when it is large enough.
  auto scratch_for = [&](size_t bytes, WsLock& ws, const char* what) -> int {
    if (!fixed) return lock_workspace(ds, s, bytes, ws, what);
    if (bytes > fixed->bytes)
      return fail(HYPNO_HIP_EINVAL,
                  "%s: this call needs %zu bytes of scratch; the fixed scratch array holds %zu",
                  what, bytes, fixed->bytes);
    ws.p = fixed->ptr;
    return HYPNO_HIP_OK;
  };
  hipError_t e;
  // Two x rows, three on a matrix of at most 16M weights: one pass of the
  // streaming GEMV with every block multiplied by each row (measured faster
  // than the few-token kernel's launches there; slower beyond, where the dot
  // products, which grow with the rows, bound it).  At four rows the
  // few-token kernel wins or ties on the Mistral-7B and TinyLlama shapes
  // (k/v 7.8 against 8.3 and 5.9 against 6.8 us per call, TinyLlama gate/up
  // 8.7 against 9.3) but for TinyLlama q/o (7.7 against 7.5).
  const bool few_rows = batch == 2 || (batch == 3 && n * m <= ((size_t)16 << 20));
  if (batch >= 2 && few_rows && q4_0_gemv_rows_ok(w, w_len, n, m, batch) && aligned16(x)) {
    e = launch_q4_0_gemv_rows(y, w, x, bias, n, m, (int)batch, cus, s);
    if (e != hipSuccess) return hip_fail(e, "q4_0 few-row GEMV launch");
    return HYPNO_HIP_OK;
  }
  if (batch >= 2 && batch <= kSkinnyMaxBatch && q4_0_skinny_ok(w, w_len, n, m, batch, cus) &&
      aligned16(x)) {
    WsLock ws;
    st = scratch_for(skinny_workspace_bytes(batch, n, m, cus), ws, "skinny workspace");
    if (st) return st;
    e = launch_q4_0_skinny(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "q4_0 skinny launch");
    return HYPNO_HIP_OK;
  }
  if (batch >= kGemmMinBatch && !gemm_folded() && q4_0_gemm_exact_ok(w, w_len, n, m, batch)) {
    WsLock ws;
    st = scratch_for(q4_0_gemm_exact_workspace_bytes(batch, n, m, cus), ws, "GEMM workspace");
    if (st) return st;
    e = launch_q4_0_gemm_exact(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "q4_0 exact GEMM launch");
    return HYPNO_HIP_OK;
  }
  const bool v3 = batch >= kGemmMinBatch && q4_0_gemm_v3_ok(w, w_len, n, m, batch);
  if (v3 || (batch >= kGemmMinBatch && q4_0_gemm_ok(w, w_len, n, m, batch))) {
    WsLock ws;
    st = scratch_for(
        v3 ? gemm_v3_workspace_bytes(batch, n, m, cus) : gemm_workspace_bytes(batch, m), ws,
        "GEMM workspace");
    if (st) return st;
    e = v3 ? launch_q4_0_gemm_v3(y, w, x, bias, n, m, batch, ws.p, cus, s)
           : launch_q4_0_gemm(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "q4_0 GEMM launch");
    return HYPNO_HIP_OK;
  }
  if (q4_0_gemv_fast_ok(w, w_len, n, m) && aligned16(x)) {
    for (size_t t = 0; t < batch; t++) {
      e = launch_q4_0_gemv_fast(y + t * n, w, x + t * m, bias, n, m, cus, s);
      if (e != hipSuccess) return hip_fail(e, "q4_0 GEMV launch");
    }
    return HYPNO_HIP_OK;
  }
  e = launch_q4_0_generic(y, w, w_len, x, bias, n, m, batch, s);
  if (e != hipSuccess) return hip_fail(e, "q4_0 generic launch");
  return HYPNO_HIP_OK;
}

// Q8_0 (ops.rs:33-36, turbo.rs:334-341): the reference dequantises the
// whole tensor and slices rows of it, so a buffer shorter than n*m elements
// is a panic there (EINVAL here).  From 16 tokens the fp16 GEMM path runs
// (weights expanded to fp16 once per call); 2 to 15 go through the few-row
// GEMV in launches of 2 to 8 rows (the tokens split evenly), one token
// through the GEMV.
int q8_0_dev(float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
             size_t n, size_t m, size_t batch, hipStream_t s) {
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  if (!y || !x) return fail(HYPNO_HIP_EINVAL, "y and x must not be NULL");
  if (mul_overflows(n, batch) || mul_overflows(m, batch) || mul_overflows(n, m))
    return fail(HYPNO_HIP_EINVAL, "shape overflows size_t");
  if (w_len / kQ8BlockBytes * kBlockElems < n * m)
    return fail(HYPNO_HIP_EINVAL, "Q8_0 weights: %zu bytes hold fewer than n*m = %zu elements",
                w_len, n * m);
  if (!w && n * m) return fail(HYPNO_HIP_EINVAL, "w is NULL");
  int st = check_disjoint(y, n * batch * 4, w, w_len, x, m * batch * 4, bias, bias ? n * 4 : 0);
  if (st) return st;
  int cus = 256;
  DeviceState* ds = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    st = device_state(&ds);
    if (st) return st;
    cus = ds->cus;
  }
  hipError_t e;
  if (batch >= kGemmMinBatch && q8_0_gemm_ok(n, m, batch)) {
    WsLock ws;
    st = lock_workspace(ds, s, q8_0_gemm_workspace_bytes(batch, n, m, cus), ws,
                        "Q8_0 GEMM workspace");
    if (st) return st;
    e = launch_q8_0_gemm(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "q8_0 GEMM launch");
    return HYPNO_HIP_OK;
  }
  const size_t launches = (batch + kQ8GemvMaxRows - 1) / kQ8GemvMaxRows;
  if (batch >= 2 && q8_0_gemv_rows_ok(w, w_len, n, m, (batch + launches - 1) / launches) &&
      aligned16(x)) {
    for (size_t c = 0, t0 = 0; c < launches; c++) {
      const size_t t1 = batch * (c + 1) / launches;  // 2..8 rows each
      e = launch_q8_0_gemv_rows(y + t0 * n, w, x + t0 * m, bias, n, m, (int)(t1 - t0), cus, s);
      if (e != hipSuccess) return hip_fail(e, "q8_0 few-row GEMV launch");
      t0 = t1;
    }
    return HYPNO_HIP_OK;
  }
  if (q8_0_gemv_fast_ok(w, w_len, n, m) && aligned16(x)) {
    for (size_t t = 0; t < batch; t++) {
      e = launch_q8_0_gemv_fast(y + t * n, w, x + t * m, bias, n, m, cus, s);
      if (e != hipSuccess) return hip_fail(e, "q8_0 GEMV launch");
    }
    return HYPNO_HIP_OK;
  }
  e = launch_q8_0_generic(y, w, x, bias, n, m, batch, s);
  if (e != hipSuccess) return hip_fail(e, "q8_0 generic launch");
  return HYPNO_HIP_OK;
}

// Column-major Q4_0 (kernels.rs:403-535): each token's product as
// turbo.rs:322-326 computes it token by token, the tokens run in groups.
int q4_0_col_dev(float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
                 size_t n, size_t m, size_t batch, hipStream_t s) {
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  if (!y || (!x && m)) return fail(HYPNO_HIP_EINVAL, "y and x must not be NULL");
  if (!w && w_len) return fail(HYPNO_HIP_EINVAL, "w_q is NULL but w_len > 0");
  // (m below 2^31 - 2^16: the kernel's k loop steps up to 128 rows past a range)
  if (mul_overflows(n, batch) || mul_overflows(m, batch) || m > 0x7FFF0000 ||
      n / kBlockElems > 0x7FFFFFFF)
    return fail(HYPNO_HIP_EINVAL, "shape out of range");
  int st = check_disjoint(y, n * batch * 4, w, w_len, x, m * batch * 4, bias, bias ? n * 4 : 0);
  if (st) return st;
  int cus = 256;
  DeviceState* ds = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    st = device_state(&ds);
    if (st) return st;
    cus = ds->cus;
  }
  // Tokens go in groups (one main and one reduction launch each) whose
  // partial planes fit 64 MB of workspace, at most 256 tokens a group.
  WsLock ws;
  const size_t per = q4_0_col_workspace_bytes(n, m, cus);
  size_t group = batch < 256 ? batch : 256;
  if (per && group > 1 && per * group > ((size_t)64 << 20))
    group = ((size_t)64 << 20) / per > 1 ? ((size_t)64 << 20) / per : 1;
  hipError_t e;
  if (per) {
    st = lock_workspace(ds, s, per * group, ws, "column-major workspace");
    if (st) return st;
  }
  for (size_t t = 0; t < batch; t += group) {
    const size_t cnt = batch - t < group ? batch - t : group;
    e = launch_q4_0_col(y + t * n, w, w_len, x + t * m, bias, n, m, (int)cnt, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "column-major Q4_0 launch");
  }
  return HYPNO_HIP_OK;
}

int f16_dev(float* y, const uint8_t* w, size_t w_len, const float* x, const float* bias,
            size_t n, size_t m, size_t batch, hipStream_t s) {
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  if (!y || !x) return fail(HYPNO_HIP_EINVAL, "y and x must not be NULL");
  if (mul_overflows(n, m) || mul_overflows(n * m, 2) || mul_overflows(n, batch) ||
      mul_overflows(m, batch))
    return fail(HYPNO_HIP_EINVAL, "shape overflows size_t");
  // kernels.rs:550 slices w16[r*m..(r+1)*m]: a short buffer is a panic there.
  if (w_len < 2 * n * m)
    return fail(HYPNO_HIP_EINVAL, "fp16 weights: w_len %zu < 2*n*m = %zu", w_len, 2 * n * m);
  if (!w && n * m) return fail(HYPNO_HIP_EINVAL, "w is NULL");
  int st = check_disjoint(y, n * batch * 4, w, w_len, x, m * batch * 4, bias, bias ? n * 4 : 0);
  if (st) return st;
  int cus = 256;
  DeviceState* ds = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    st = device_state(&ds);
    if (st) return st;
    cus = ds->cus;
  }
  hipError_t e;
  if (f16_gemm_stream_ok(w, x, n, m, batch)) {
    WsLock ws;
    st = lock_workspace(ds, s, f16_gemm_stream_workspace_bytes(batch, n, m, cus), ws,
                        "GEMM workspace");
    if (st) return st;
    e = launch_f16_gemm_stream(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "f16 GEMM launch");
    return HYPNO_HIP_OK;
  }
  if (batch >= kGemmMinBatch && f16_gemm_v2_ok(w, n, m, batch)) {
    WsLock ws;
    st = lock_workspace(ds, s, f16_gemm_v2_workspace_bytes(batch, n, m, cus), ws,
                        "GEMM workspace");
    if (st) return st;
    e = launch_f16_gemm_v2(y, w, x, bias, n, m, batch, ws.p, cus, s);
    if (e != hipSuccess) return hip_fail(e, "f16 GEMM launch");
    return HYPNO_HIP_OK;
  }
  if (f16_gemv_fast_ok(w, n, m) && aligned16(x)) {
    for (size_t t = 0; t < batch; t++) {
      e = launch_f16_gemv_fast(y + t * n, w, x + t * m, bias, n, m, cus, s);
      if (e != hipSuccess) return hip_fail(e, "f16 GEMV launch");
    }
    return HYPNO_HIP_OK;
  }
  e = launch_f16_generic(y, w, x, bias, n, m, batch, s);
  if (e != hipSuccess) return hip_fail(e, "f16 generic launch");
  return HYPNO_HIP_OK;
}

// --- host-slice path ----------------------------------------------------------

int host_matmul(float* y, const uint8_t* w, size_t w_len, uint32_t dtype, const float* x,
                const float* bias, size_t n, size_t m, size_t batch, bool col = false) {
  if (dtype == HYPNO_DTYPE_FP32)
    return fail(HYPNO_HIP_ENOTSUP, "dtype %u is not on the quantised/FP16 path", dtype);
  if (dtype != HYPNO_DTYPE_Q4_0 && dtype != HYPNO_DTYPE_FP16 && dtype != HYPNO_DTYPE_Q8_0)
    return fail(HYPNO_HIP_EINVAL, "unknown dtype %u", dtype);
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  if (!y || (!x && m) || (!w && w_len))
    return fail(HYPNO_HIP_EINVAL, "NULL pointer argument");
  if (mul_overflows(n, batch) || mul_overflows(m, batch) || mul_overflows(n * batch, 4) ||
      mul_overflows(m * batch, 4))
    return fail(HYPNO_HIP_EINVAL, "shape overflows size_t");
  if (dtype == HYPNO_DTYPE_FP16 && (mul_overflows(n, m) || w_len < 2 * n * m))
    return fail(HYPNO_HIP_EINVAL, "fp16 weights: w_len %zu < 2*n*m", w_len);
  if (dtype == HYPNO_DTYPE_Q8_0 &&
      (mul_overflows(n, m) || w_len / kQ8BlockBytes * kBlockElems < n * m))
    return fail(HYPNO_HIP_EINVAL, "Q8_0 weights: %zu bytes hold fewer than n*m elements", w_len);

  // One host-slice call at a time: the staging buffers and the registry's
  // device copies are shared by all callers.
  std::lock_guard<std::mutex> hg(g_host_mu);
  DeviceState* ds = nullptr;
  int dev = 0;
  const uint8_t* dw = nullptr;
  bool resident = false;
  {
    std::lock_guard<std::mutex> g(g_mu);
    int st = device_state(&ds);
    if (st) return st;
    (void)hipGetDevice(&dev);
    auto it = g_weights.find(w);
    if (it != g_weights.end() && it->second.len == w_len && it->second.device == dev) {
      dw = (const uint8_t*)it->second.dev_ptr;
      resident = true;
    }
  }
  hipStream_t s = ds->stream;
  hipError_t e;
  int st;

  if (!resident && w_len) {
    if ((e = ensure(ds->w, w_len, s)) != hipSuccess) return hip_fail(e, "weight staging");
    if ((e = hipMemcpyAsync(ds->w.p, w, w_len, hipMemcpyHostToDevice, s)) != hipSuccess)
      return hip_fail(e, "weight upload");
    dw = (const uint8_t*)ds->w.p;
  }
  const size_t xb = m * batch * 4, yb = n * batch * 4;
  if ((e = ensure(ds->x, xb, s)) != hipSuccess) return hip_fail(e, "x staging");
  if ((e = ensure(ds->y, yb, s)) != hipSuccess) return hip_fail(e, "y staging");
  // Every call ends with the stream drained, so the page-locked buffers are
  // free again when the next call (serialised by g_host_mu) fills them.
  if (xb && (e = upload(ds->x.p, x, xb, ds->hx, s)) != hipSuccess) return hip_fail(e, "x upload");
  const bool ypin = yb <= kPinnedMax;
  if (ypin && (e = ensure_host(ds->hy, yb, s)) != hipSuccess) return hip_fail(e, "y staging");
  // One token, row-major: the GEMV writes y straight into the mapped
  // page-locked buffer (plain stores of finished rows, nothing read back),
  // which saves the device-to-host copy.
  float* dy = (float*)ds->y.p;
  bool ydirect = false;
  if (ypin && batch == 1 && !col) {
    void* dp = nullptr;
    if (hipHostGetDevicePointer(&dp, ds->hy.p, 0) == hipSuccess && dp) {
      dy = (float*)dp;
      ydirect = true;
    }
  }
  float* db = nullptr;
  if (bias) {
    if ((e = ensure(ds->bias, n * 4, s)) != hipSuccess) return hip_fail(e, "bias staging");
    if ((e = upload(ds->bias.p, bias, n * 4, ds->hbias, s)) != hipSuccess)
      return hip_fail(e, "bias upload");
    db = (float*)ds->bias.p;
  }
  if (dtype == HYPNO_DTYPE_Q4_0 && col)
    st = q4_0_col_dev(dy, dw, w_len, (const float*)ds->x.p, db, n, m, batch, s);
  else if (dtype == HYPNO_DTYPE_Q4_0)
    st = q4_0_dev(dy, dw, w_len, (const float*)ds->x.p, db, n, m, batch, s);
  else if (dtype == HYPNO_DTYPE_Q8_0)
    st = q8_0_dev(dy, dw, w_len, (const float*)ds->x.p, db, n, m, batch, s);
  else
    st = f16_dev(dy, dw, w_len, (const float*)ds->x.p, db, n, m, batch, s);
  if (st) {
    (void)hipStreamSynchronize(s);
    return st;
  }
  if (!ydirect &&
      (e = hipMemcpyAsync(ypin ? ds->hy.p : y, ds->y.p, yb, hipMemcpyDeviceToHost, s)) !=
          hipSuccess) {
    (void)hipStreamSynchronize(s);
    return hip_fail(e, "y download");
  }
  if ((e = hipStreamSynchronize(s)) != hipSuccess) return hip_fail(e, "stream synchronize");
  if (ypin && yb) memcpy(y, ds->hy.p, yb);
  return HYPNO_HIP_OK;
}

}  // namespace

namespace hypno {

int set_last_error(int status, const std::string& msg) {
  g_last_error = msg;
  return status;
}

int hip_status(hipError_t e, const char* what) { return hip_fail(e, what); }

static std::atomic<uint32_t> g_gemm_numerics{HYPNO_HIP_GEMM_AUTO};

bool gemm_folded() { return g_gemm_numerics.load() == HYPNO_HIP_GEMM_FOLDED; }

hipError_t set_lds_limit(const void* kernel, int bytes) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> g(mu);
  if (done.count({kernel, dev})) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert({kernel, dev});
  return e;
}

}  // namespace hypno

namespace {

// Scratch memory of the no-allocation entry point: one fixed array per GPU
// (every device the library runs on holds its own copy until the process
// ends).  Host code never uses the array's name as an address: the device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and is kept in g_scratch.
constexpr size_t kScratchBytes = HYPNO_HIP_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
FixedScratch g_scratch[kMaxDevices];

int scratch_of_current_device(FixedScratch* out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(HYPNO_HIP_EINVAL, "device %d: the no-allocation path supports %d devices", dev,
                kMaxDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  FixedScratch& sc = g_scratch[dev];
  if (!sc.ptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(HYPNO_HIP_EDEVICE, "hipGetSymbolAddress(scratch) gave NULL");
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    sc.cus = cus;
    sc.bytes = kScratchBytes;
    sc.ptr = p;
  }
  *out = sc;
  return HYPNO_HIP_OK;
}

}  // namespace

extern "C" {

int hypno_hip_abi_version(void) { return HYPNO_HIP_ABI_VERSION; }

const char* hypno_hip_strerror(int status) {
  switch (status) {
    case HYPNO_HIP_OK: return "ok";
    case HYPNO_HIP_EINVAL: return "invalid argument";
    case HYPNO_HIP_ENOMEM: return "out of memory";
    case HYPNO_HIP_EDEVICE: return "device or HIP runtime error";
    case HYPNO_HIP_ENOTSUP: return "dtype not supported on this path";
    case HYPNO_HIP_ENOENT: return "no such file, tensor or metadata key";
    case HYPNO_HIP_EFILE: return "file could not be opened, mapped or read";
    case HYPNO_HIP_EFORMAT: return "malformed .hypno file";
    default: return "unknown status";
  }
}

const char* hypno_hip_last_error(void) { return g_last_error.c_str(); }

int hypno_hip_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  return n;
}

int hypno_hip_matmul_q4_0(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                          const float* bias, size_t n, size_t m) {
  return host_matmul(y, w_q, w_len, HYPNO_DTYPE_Q4_0, x, bias, n, m, 1);
}

int hypno_hip_matmul_f16(float* y, const uint8_t* w, size_t w_len, const float* x,
                         const float* bias, size_t n, size_t m) {
  return host_matmul(y, w, w_len, HYPNO_DTYPE_FP16, x, bias, n, m, 1);
}

int hypno_hip_matmul_q8_0(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                          const float* bias, size_t n, size_t m) {
  return host_matmul(y, w_q, w_len, HYPNO_DTYPE_Q8_0, x, bias, n, m, 1);
}

int hypno_hip_matmul_vec_auto(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                              const float* x, const float* bias, size_t n, size_t m) {
  return host_matmul(y, w, w_len, dtype, x, bias, n, m, 1);
}

int hypno_hip_batch_matmul(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                           const float* x, size_t n, size_t dim, size_t batch) {
  return host_matmul(y, w, w_len, dtype, x, nullptr, n, dim, batch);
}

int hypno_hip_matmul_q4_0_col(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m) {
  return host_matmul(y, w_q, w_len, HYPNO_DTYPE_Q4_0, x, bias, n, m, 1, true);
}

int hypno_hip_matmul_vec_col(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                             const float* x, const float* bias, size_t n, size_t m) {
  return host_matmul(y, w, w_len, dtype, x, bias, n, m, 1, true);
}

int hypno_hip_batch_matmul_col(float* y, const uint8_t* w, size_t w_len, uint32_t dtype,
                               const float* x, size_t n, size_t dim, size_t batch) {
  return host_matmul(y, w, w_len, dtype, x, nullptr, n, dim, batch, true);
}

int hypno_hip_matmul_q4_0_col_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                                  const float* bias, size_t n, size_t m, size_t batch,
                                  void* stream) {
  return q4_0_col_dev(y, w_q, w_len, x, bias, n, m, batch, (hipStream_t)stream);
}

int hypno_hip_weight_register(const uint8_t* host, size_t len) {
  if (!host || !len) return fail(HYPNO_HIP_EINVAL, "register: NULL or empty buffer");
  std::lock_guard<std::mutex> hg(g_host_mu);
  std::lock_guard<std::mutex> g(g_mu);
  DeviceState* ds = nullptr;
  int st = device_state(&ds);
  if (st) return st;
  int dev = 0;
  (void)hipGetDevice(&dev);
  auto it = g_weights.find(host);
  if (it != g_weights.end()) {
    if (it->second.len == len && it->second.device == dev) return HYPNO_HIP_OK;
    (void)hipFree(it->second.dev_ptr);
    g_weights.erase(it);
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, len);
  if (e != hipSuccess) return hip_fail(e, "register: hipMalloc");
  e = hipMemcpy(p, host, len, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "register: upload");
  }
  g_weights[host] = Registered{p, len, dev};
  return HYPNO_HIP_OK;
}

int hypno_hip_weight_unregister(const uint8_t* host) {
  std::lock_guard<std::mutex> hg(g_host_mu);
  std::lock_guard<std::mutex> g(g_mu);
  auto it = g_weights.find(host);
  if (it == g_weights.end()) return fail(HYPNO_HIP_EINVAL, "unregister: pointer not registered");
  (void)hipDeviceSynchronize();
  (void)hipFree(it->second.dev_ptr);
  g_weights.erase(it);
  return HYPNO_HIP_OK;
}

int hypno_hip_matmul_q4_0_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m, size_t batch,
                              void* stream) {
  return q4_0_dev(y, w_q, w_len, x, bias, n, m, batch, (hipStream_t)stream);
}

int hypno_hip_matmul_q4_0_dev_noalloc(float* y, const uint8_t* w_q, size_t w_len,
                                      const float* x, const float* bias, size_t n, size_t m,
                                      size_t batch, void* stream) {
  if (n == 0 || batch == 0) return HYPNO_HIP_OK;
  FixedScratch sc;
  int st = scratch_of_current_device(&sc);
  if (st) return st;
  return q4_0_dev(y, w_q, w_len, x, bias, n, m, batch, (hipStream_t)stream, &sc);
}

int hypno_hip_matmul_f16_dev(float* y, const uint8_t* w, size_t w_len, const float* x,
                             const float* bias, size_t n, size_t m, size_t batch, void* stream) {
  return f16_dev(y, w, w_len, x, bias, n, m, batch, (hipStream_t)stream);
}

int hypno_hip_matmul_q8_0_dev(float* y, const uint8_t* w_q, size_t w_len, const float* x,
                              const float* bias, size_t n, size_t m, size_t batch,
                              void* stream) {
  return q8_0_dev(y, w_q, w_len, x, bias, n, m, batch, (hipStream_t)stream);
}

int hypno_hip_quantize_q8_0_dev(uint8_t* out, const float* src, size_t n_elems, void* stream) {
  const size_t nb = n_elems / kBlockElems;
  if (nb == 0) return HYPNO_HIP_OK;
  if (!out || !src) return fail(HYPNO_HIP_EINVAL, "quantize: NULL pointer");
  hipError_t e = launch_quantize_q8_0(out, src, nb, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantize launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_dequantize_q8_0_dev(float* out, const uint8_t* q, size_t q_len, void* stream) {
  const size_t nb = q_len / kQ8BlockBytes;
  if (nb == 0) return HYPNO_HIP_OK;
  if (!out || !q) return fail(HYPNO_HIP_EINVAL, "dequantize: NULL pointer");
  hipError_t e = launch_dequantize_q8_0(out, q, nb, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_quantize_q4_0_dev(uint8_t* out, const float* src, size_t n_elems, void* stream) {
  const size_t nb = n_elems / kBlockElems;
  if (nb == 0) return HYPNO_HIP_OK;
  if (!out || !src) return fail(HYPNO_HIP_EINVAL, "quantize: NULL pointer");
  hipError_t e = launch_quantize_q4_0(out, src, nb, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "quantize launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_dequantize_q4_0_dev(float* out, const uint8_t* q, size_t q_len, void* stream) {
  const size_t nb = q_len / kBlockBytes;
  if (nb == 0) return HYPNO_HIP_OK;
  if (!out || !q) return fail(HYPNO_HIP_EINVAL, "dequantize: NULL pointer");
  hipError_t e = launch_dequantize_q4_0(out, q, nb, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "dequantize launch");
  return HYPNO_HIP_OK;
}

}  // extern "C"

struct hypno_hip_gemv_plan {
  struct Group {
    GemvGroupGeom geom;
    GemvJob* d_jobs = nullptr;  // device table (njobs > kGemvInline)
    GemvJob inl[kGemvInline];   // the first jobs (all of them up to kGemvInline)
    int njobs = 0;
    int total_steps = 0;
  };
  // A job the streaming kernel cannot take: the any-shape kernel, after a
  // stand-alone prologue into `staged` when the job has one.
  struct Generic {
    hypno_hip_gemv_desc d;
    hypno_hip_gemv_prologue pro;
    float* staged = nullptr;  // [m], plan-owned
  };
  int device = 0;
  int cus = 256;
  std::vector<Group> groups;
  std::vector<Generic> generic;
};

namespace {

int close_group(hypno_hip_gemv_plan* pl, hypno_hip_gemv_plan::Group& grp,
                std::vector<GemvJob>& jobs) {
  if (jobs.empty()) return HYPNO_HIP_OK;
  {
    std::vector<int> ns, bs;
    for (const GemvJob& j : jobs) {
      ns.push_back(j.n);
      bs.push_back(j.B);
    }
    gemv_group_widen(grp.geom, ns.data(), bs.data(), (int)jobs.size(), pl->cus);
  }
  long long step = 0;
  for (GemvJob& j : jobs) {
    j.rps = grp.geom.T / j.B;
    j.step0 = (int)step;
    step += (j.n + j.rps - 1) / j.rps;
  }
  if (step > 0x7FFFFFFF) return fail(HYPNO_HIP_EINVAL, "plan: too many rows in one group");
  grp.njobs = (int)jobs.size();
  grp.total_steps = (int)step;
  for (int i = 0; i < kGemvInline && i < grp.njobs; i++) grp.inl[i] = jobs[i];
  if (grp.njobs > kGemvInline) {
    hipError_t e = hipMalloc(&grp.d_jobs, jobs.size() * sizeof(GemvJob));
    if (e != hipSuccess) return hip_fail(e, "plan: job table");
    e = hipMemcpy(grp.d_jobs, jobs.data(), jobs.size() * sizeof(GemvJob), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(grp.d_jobs);
      grp.d_jobs = nullptr;
      return hip_fail(e, "plan: job table upload");
    }
  }
  pl->groups.push_back(grp);
  grp = hypno_hip_gemv_plan::Group();
  jobs.clear();
  return HYPNO_HIP_OK;
}

// The jobs of a plan run concurrently in one launch: no job's y may share
// memory with another job's y, nor with any job's inputs (x, w, bias and the
// prologue operand aux).  Sorted write ranges make this O(count log count).
int check_plan_disjoint(const hypno_hip_gemv_desc* descs, const hypno_hip_gemv_prologue* pros,
                        size_t count) {
  struct Range {
    uintptr_t a, b;
    size_t job;
  };
  std::vector<Range> writes, reads;
  auto add = [](std::vector<Range>& v, const void* p, size_t bytes, size_t job) {
    if (p && bytes) v.push_back({(uintptr_t)p, (uintptr_t)p + bytes, job});
  };
  for (size_t i = 0; i < count; i++) {
    const hypno_hip_gemv_desc& d = descs[i];
    if (d.n == 0) continue;
    if (mul_overflows(d.n, 4) || mul_overflows(d.m, 4))
      return fail(HYPNO_HIP_EINVAL, "plan_create: descriptor %zu shape overflows", i);
    add(writes, d.y, d.n * 4, i);
    add(reads, d.x, d.m * 4, i);
    add(reads, d.w_q, d.w_len, i);
    add(reads, d.bias, d.n * 4, i);
    if (pros && pros[i].kind != HYPNO_HIP_PROLOGUE_NONE) add(reads, pros[i].aux, d.m * 4, i);
  }
  std::sort(writes.begin(), writes.end(),
            [](const Range& p, const Range& q) { return p.a < q.a; });
  for (size_t i = 1; i < writes.size(); i++)
    if (writes[i].a < writes[i - 1].b)
      return fail(HYPNO_HIP_EINVAL, "plan_create: y of descriptors %zu and %zu overlap",
                  writes[i - 1].job, writes[i].job);
  for (const Range& r : reads) {
    // first write range ending after r starts (ends are sorted like starts)
    auto it = std::lower_bound(writes.begin(), writes.end(), r.a,
                               [](const Range& w, uintptr_t a) { return w.b <= a; });
    if (it != writes.end() && it->a < r.b)
      return fail(HYPNO_HIP_EINVAL,
                  "plan_create: y of descriptor %zu overlaps an input of descriptor %zu", it->job,
                  r.job);
  }
  return HYPNO_HIP_OK;
}

void free_plan(hypno_hip_gemv_plan* pl) {
  for (auto& g : pl->groups)
    if (g.d_jobs) (void)hipFree(g.d_jobs);
  for (auto& g : pl->generic)
    if (g.staged) (void)hipFree(g.staged);
  delete pl;
}

}  // namespace

extern "C" {

int hypno_hip_q4_0_gemv_plan_create(const hypno_hip_gemv_desc* descs, size_t count,
                                    hypno_hip_gemv_plan** plan) {
  return hypno_hip_q4_0_gemv_plan_create_ex(descs, nullptr, count, plan);
}

int hypno_hip_q4_0_gemv_plan_create_ex(const hypno_hip_gemv_desc* descs,
                                       const hypno_hip_gemv_prologue* prologues, size_t count,
                                       hypno_hip_gemv_plan** plan) {
  if (!plan) return fail(HYPNO_HIP_EINVAL, "plan_create: NULL plan pointer");
  *plan = nullptr;
  if (!descs && count) return fail(HYPNO_HIP_EINVAL, "plan_create: NULL descriptors");
  {
    int st = check_plan_disjoint(descs, prologues, count);
    if (st) return st;
  }
  int cus = 256;
  {
    std::lock_guard<std::mutex> g(g_mu);
    DeviceState* ds = nullptr;
    int st = device_state(&ds);
    if (st) return st;
    cus = ds->cus;
  }
  hypno_hip_gemv_plan* pl = new hypno_hip_gemv_plan();
  (void)hipGetDevice(&pl->device);
  pl->cus = cus;
  hypno_hip_gemv_plan::Group grp;
  std::vector<GemvJob> jobs;
  for (size_t i = 0; i < count; i++) {
    const hypno_hip_gemv_desc& d = descs[i];
    if (d.n == 0) continue;
    if (!d.y || !d.x || (!d.w_q && d.w_len)) {
      free_plan(pl);
      return fail(HYPNO_HIP_EINVAL, "plan_create: descriptor %zu has a NULL pointer", i);
    }
    if (mul_overflows(d.n, d.m)) {
      free_plan(pl);
      return fail(HYPNO_HIP_EINVAL, "plan_create: descriptor %zu shape overflows", i);
    }
    hypno_hip_gemv_prologue pro = {HYPNO_HIP_PROLOGUE_NONE, nullptr, 0.0f};
    if (prologues) pro = prologues[i];
    if (pro.kind > HYPNO_HIP_PROLOGUE_SILU_MUL) {
      free_plan(pl);
      return fail(HYPNO_HIP_EINVAL, "plan_create: descriptor %zu has unknown prologue %u", i,
                  pro.kind);
    }
    if (pro.kind != HYPNO_HIP_PROLOGUE_NONE && (!pro.aux || d.m == 0)) {
      free_plan(pl);
      return fail(HYPNO_HIP_EINVAL, "plan_create: descriptor %zu: prologue needs aux and m > 0",
                  i);
    }
    if (!(q4_0_gemv_fast_ok(d.w_q, d.w_len, d.n, d.m) && aligned16(d.x) &&
          (pro.kind == HYPNO_HIP_PROLOGUE_NONE || aligned16(pro.aux)))) {
      hypno_hip_gemv_plan::Generic gj;
      gj.d = d;
      gj.pro = pro;
      if (pro.kind != HYPNO_HIP_PROLOGUE_NONE) {
        hipError_t e = hipMalloc(&gj.staged, d.m * sizeof(float));
        if (e != hipSuccess) {
          free_plan(pl);
          return hip_fail(e, "plan_create: prologue staging");
        }
      }
      pl->generic.push_back(gj);
      continue;
    }
    if (!gemv_group_add(grp.geom, d.m)) {
      int st = close_group(pl, grp, jobs);
      if (st) {
        free_plan(pl);
        return st;
      }
      gemv_group_add(grp.geom, d.m);
    }
    if (pro.kind != HYPNO_HIP_PROLOGUE_NONE) grp.geom.pro = 1;
    GemvJob j;
    j.w = d.w_q;
    j.x = d.x;
    j.y = d.y;
    j.bias = d.bias;
    j.aux = pro.aux;
    j.pro = (int)pro.kind;
    j.eps = pro.eps;
    j.n = (int)d.n;
    j.B = (int)(d.m / 32);
    j.rps = 0;
    j.step0 = 0;
    jobs.push_back(j);
  }
  int st = close_group(pl, grp, jobs);
  if (st) {
    free_plan(pl);
    return st;
  }
  *plan = pl;
  return HYPNO_HIP_OK;
}

int hypno_hip_q4_0_gemv_plan_run(const hypno_hip_gemv_plan* plan, void* stream) {
  if (!plan) return fail(HYPNO_HIP_EINVAL, "plan_run: NULL plan");
  hipStream_t s = (hipStream_t)stream;
  for (const auto& g : plan->groups) {
    hipError_t e = launch_q4_0_gemv_group(g.geom, g.d_jobs, g.inl, g.njobs, g.total_steps,
                                          plan->cus, s);
    if (e != hipSuccess) return hip_fail(e, "plan_run: GEMV launch");
  }
  for (const auto& g : plan->generic) {
    const hypno_hip_gemv_desc& d = g.d;
    const float* x = d.x;
    hipError_t e = hipSuccess;
    if (g.pro.kind == HYPNO_HIP_PROLOGUE_RMS_NORM)
      e = launch_rms_norm(g.staged, d.x, g.pro.aux, d.m, 1, g.pro.eps, s);
    else if (g.pro.kind == HYPNO_HIP_PROLOGUE_SILU_MUL)
      e = launch_silu_mul(g.staged, d.x, g.pro.aux, d.m, s);
    if (e != hipSuccess) return hip_fail(e, "plan_run: prologue launch");
    if (g.staged) x = g.staged;
    e = launch_q4_0_generic(d.y, d.w_q, d.w_len, x, d.bias, d.n, d.m, 1, s);
    if (e != hipSuccess) return hip_fail(e, "plan_run: generic launch");
  }
  return HYPNO_HIP_OK;
}

int hypno_hip_q4_0_gemv_plan_launches(const hypno_hip_gemv_plan* plan) {
  if (!plan) return 0;
  int n = (int)(plan->groups.size() + plan->generic.size());
  for (const auto& g : plan->generic) n += g.staged ? 1 : 0;
  return n;
}

int hypno_hip_q4_0_gemv_plan_destroy(hypno_hip_gemv_plan* plan) {
  if (!plan) return HYPNO_HIP_OK;
  (void)hipDeviceSynchronize();
  free_plan(plan);
  return HYPNO_HIP_OK;
}

int hypno_hip_rms_norm_dev(float* out, const float* x, const float* weight, size_t n,
                           size_t rows, float eps, void* stream) {
  if (n == 0 || rows == 0) return HYPNO_HIP_OK;
  if (!out || !x || !weight) return fail(HYPNO_HIP_EINVAL, "rms_norm: NULL pointer");
  if (mul_overflows(n, rows) || rows > 0x7FFFFFFF)
    return fail(HYPNO_HIP_EINVAL, "rms_norm: shape overflows");
  hipError_t e = launch_rms_norm(out, x, weight, n, rows, eps, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "rms_norm launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_silu_mul_dev(float* out, const float* gate, const float* up, size_t n,
                           void* stream) {
  if (n == 0) return HYPNO_HIP_OK;
  if (!out || !gate || !up) return fail(HYPNO_HIP_EINVAL, "silu_mul: NULL pointer");
  hipError_t e = launch_silu_mul(out, gate, up, n, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "silu_mul launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_q4_0_extract_row_dev(float* out, const uint8_t* q, size_t q_len, size_t row_idx,
                                   size_t row_width, void* stream) {
  if (row_width == 0) return HYPNO_HIP_OK;
  if (!out) return fail(HYPNO_HIP_EINVAL, "extract_row: NULL output");
  const size_t bpr = row_width / kBlockElems;
  if (bpr && (mul_overflows(row_idx + 1, bpr * kBlockBytes) || !q ||
              (row_idx + 1) * bpr * kBlockBytes > q_len))
    return fail(HYPNO_HIP_EINVAL, "extract_row: row %zu is past the end of the %zu-byte matrix",
                row_idx, q_len);
  hipError_t e = launch_embed_rows(out, q, q_len, (int)HYPNO_DTYPE_Q4_0, nullptr, row_idx, 1,
                                   row_width, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "extract_row launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_q8_0_extract_row_dev(float* out, const uint8_t* q, size_t q_len, size_t row_idx,
                                   size_t row_width, void* stream) {
  if (row_width == 0) return HYPNO_HIP_OK;
  if (!out) return fail(HYPNO_HIP_EINVAL, "extract_row: NULL output");
  const size_t bpr = row_width / kBlockElems;
  if (bpr && (mul_overflows(row_idx + 1, bpr * kQ8BlockBytes) || !q ||
              (row_idx + 1) * bpr * kQ8BlockBytes > q_len))
    return fail(HYPNO_HIP_EINVAL, "extract_row: row %zu is past the end of the %zu-byte matrix",
                row_idx, q_len);
  hipError_t e = launch_embed_rows(out, q, q_len, (int)HYPNO_DTYPE_Q8_0, nullptr, row_idx, 1,
                                   row_width, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "extract_row launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_embed_tokens_dev(float* out, const uint8_t* table, size_t table_len,
                               uint32_t dtype, const uint32_t* ids, size_t count, size_t hd,
                               void* stream) {
  if (dtype > HYPNO_DTYPE_Q4_0) return fail(HYPNO_HIP_EINVAL, "embed: unknown dtype %u", dtype);
  if (count == 0 || hd == 0) return HYPNO_HIP_OK;
  if (!out || !ids || (!table && table_len)) return fail(HYPNO_HIP_EINVAL, "embed: NULL pointer");
  if (count > 0x7FFFFFFF || mul_overflows(count, hd) || hd > ((size_t)1 << 40))
    return fail(HYPNO_HIP_EINVAL, "embed: shape out of range");
  hipError_t e = launch_embed_rows(out, table, table_len, (int)dtype, ids, 0, count, hd,
                                   (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "embed launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_argmax_dev(uint32_t* index, const float* logits, size_t n, void* stream) {
  if (!index || (!logits && n)) return fail(HYPNO_HIP_EINVAL, "argmax: NULL pointer");
  if (n > 0x7FFFFFFF) return fail(HYPNO_HIP_EINVAL, "argmax: n out of range");
  hipStream_t s = (hipStream_t)stream;
  DeviceState* ds = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    int st = device_state(&ds);
    if (st) return st;
  }
  WsLock ws;
  int st = lock_workspace(ds, s, sample_workspace_bytes(n, true), ws, "argmax workspace");
  if (st) return st;
  hipError_t e = launch_sample_token(index, nullptr, logits, n, 0.0f, 1.0f, 0, true, ws.p, s);
  if (e != hipSuccess) return hip_fail(e, "argmax launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_sample_token_dev(uint32_t* token, uint64_t* rng_state, const float* logits,
                               size_t n, float temperature, float top_p, size_t top_k,
                               void* stream) {
  if (!token || !rng_state || (!logits && n))
    return fail(HYPNO_HIP_EINVAL, "sample_token: NULL pointer");
  if (n > 0x7FFFFFFF) return fail(HYPNO_HIP_EINVAL, "sample_token: n out of range");
  hipStream_t s = (hipStream_t)stream;
  DeviceState* ds = nullptr;
  {
    std::lock_guard<std::mutex> g(g_mu);
    int st = device_state(&ds);
    if (st) return st;
  }
  WsLock ws;
  int st = lock_workspace(ds, s, sample_workspace_bytes(n, false), ws, "sampling workspace");
  if (st) return st;
  hipError_t e = launch_sample_token(token, rng_state, logits, n, temperature, top_p, top_k,
                                     false, ws.p, s);
  if (e != hipSuccess) return hip_fail(e, "sample_token launch");
  return HYPNO_HIP_OK;
}

int hypno_hip_set_gemm_numerics(uint32_t mode) {
  if (mode != HYPNO_HIP_GEMM_AUTO && mode != HYPNO_HIP_GEMM_EXACT && mode != HYPNO_HIP_GEMM_FOLDED) {
    fail(HYPNO_HIP_EINVAL, "set_gemm_numerics: unknown mode %u", mode);
    return -HYPNO_HIP_EINVAL;
  }
  return (int)g_gemm_numerics.exchange(mode);
}

int hypno_hip_stream_synchronize(void* stream) {
  hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  return HYPNO_HIP_OK;
}

}  // extern "C"
